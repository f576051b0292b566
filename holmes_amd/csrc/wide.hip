// The wide-prime path (primes in (2^31, 2^61), any of them >= 2^50): every kernel of the library's
// internal entry points restated on 64-bit integer words.  Residues are canonical in [0, p) in HBM
// and between stages; products by constants (twiddles, base-conversion factors, P^-1, N^-1) use
// Shoup's precomputed quotient, products of two variables (keys, plaintexts, ciphertext tensors)
// Barrett's reduction (modarith64.hpp).  The algorithms are the FP64 path's -- two-pass negacyclic
// NTT (256 x 256, LDS-staged), hybrid key switch (ModUp by the centered fast base conversion, key
// inner product, ModDown), rescale and ModRaise by the centered lift -- and produce the same
// residues as the CPU oracle, which is exact for any prime below 2^62.
//
// The kernels favour plainness over speed: the key switch runs as separate launches (INTT, one
// conversion + NTT + inner product per digit, ModDown per component) over chunks of kWideChunk
// items with its intermediates in the workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "modarith64.hpp"
#include "wide.hpp"
#include "wide_dev.hpp"

using u64 = uint64_t;
using u128 = unsigned __int128;

namespace hck {
namespace {

// ------------------------------------------------------------------------------------ host helpers
u64 hmul(u64 a, u64 b, u64 q) { return (u64)((u128)a * b % q); }
u64 hpow(u64 b, u64 e, u64 q) {
  u64 r = 1;
  b %= q;
  while (e) {
    if (e & 1) r = hmul(r, b, q);
    b = hmul(b, b, q);
    e >>= 1;
  }
  return r;
}
u64 hinv(u64 a, u64 q) { return hpow(a % q, q - 2, q); }
u64 hbrv(u64 x, int bits) {
  u64 r = 0;
  for (int i = 0; i < bits; ++i) {
    r = (r << 1) | (x & 1);
    x >>= 1;
  }
  return r;
}

void fill_wide_conv(WideConv& cc, const std::vector<u64>& P, const std::vector<int>& src, const std::vector<int>& dst,
                    const std::vector<int>& slot) {
  std::memset(&cc, 0, sizeof(cc));
  cc.ns = (int)src.size();
  cc.nt = (int)dst.size();
  for (int s = 0; s < cc.ns; ++s) {
    const u64 bs = P[src[s]];
    u64 h = 1;
    for (int r = 0; r < cc.ns; ++r)
      if (r != s) h = hmul(h, P[src[r]] % bs, bs);
    cc.src_prime[s] = src[s];
    cc.hinv[s] = hinv(h, bs);
    cc.hinv_s[s] = shoup_companion(cc.hinv[s], bs);
    for (int t = 0; t < cc.nt; ++t) {
      const u64 qt = P[dst[t]];
      u64 v = 1;
      for (int r = 0; r < cc.ns; ++r)
        if (r != s) v = hmul(v, P[src[r]] % qt, qt);
      cc.hmod[s][t] = v;
      cc.hmod_s[s][t] = shoup_companion(v, qt);
      cc.hmod_m[s][t] = (u64)(((u128)v << 64) % qt);
    }
  }
  for (int t = 0; t < cc.nt; ++t) {
    const u64 qt = P[dst[t]];
    u64 inv = qt;  // Newton's iteration for qt^-1 mod 2^64: each step doubles the correct low bits
    for (int i = 0; i < 6; ++i) inv *= 2 - qt * inv;
    cc.tneg_inv[t] = 0 - inv;
    cc.dst_prime[t] = dst[t];
    cc.dst_slot[t] = slot[t];
  }
}

// ---------------------------------------------------------------------------------------------- NTT
// Forward transform (Cooley-Tukey, psi^brv roots, bit-reversed evaluation order out), as two passes
// (src == dst allowed: a block reads its 16 columns or rows whole before it writes them back)
// over the 256 x 256 view of a limb (element 256 r + c): the first eight stages act on the columns
// (fixed c, a 256-point transform over r with root psi_rev[m + r-group]), the last eight on the rows.
// A block holds 16 columns or 16 rows; 256 threads.  Each pass runs its eight stages as two
// radix-16 rounds in registers (16 words per thread) with one LDS exchange between them: in the
// first round a thread holds the 16 elements 16 apart, in the second the 16 consecutive ones.
constexpr int kWT = 256;
constexpr int kWPad = 17;  // LDS row stride of the column kernels (words)

__device__ __forceinline__ int wpad(int k) { return k + (k >> 4); }  // row kernels' LDS index

// Four Cooley-Tukey stages over x[0..15] at distances 8, 4, 2, 1: stage s pairs (u, u + (8 >> s))
// with root index base(s) + (group(s, u)), the caller's closure.
template <typename Root>
__device__ __forceinline__ void wfwd16(u64 (&x)[16], const u64* tw, const u64* tws, u64 p, Root root) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d = 8 >> s;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u & d) continue;
      const int wi = root(s, u);
      const u64 y = wmulc(x[u + d], tw[wi], tws[wi], p);
      const u64 a = x[u];
      x[u] = wadd(a, y, p);
      x[u + d] = wsub(a, y, p);
    }
  }
}

// Four Gentleman-Sande stages over x[0..15] at distances 1, 2, 4, 8: (a, b) -> (a + b, (a - b) w).
template <typename Root>
__device__ __forceinline__ void winv16(u64 (&x)[16], const u64* tw, const u64* tws, u64 p, Root root) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d = 1 << s;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u & d) continue;
      const int wi = root(s, u);
      const u64 a = x[u], b = x[u + d];
      x[u] = wadd(a, b, p);
      x[u + d] = wmulc(wsub(a, b, p), tw[wi], tws[wi], p);
    }
  }
}

// The same stages on lazy words (Harvey): forward butterflies take and return words below 4p, inverse
// ones below 2p (Shoup's lazy products lie below 2p for any 64-bit input; 4p < 2^63).  The NTT kernels
// below run on them and canonicalise what they store, so that their outputs stay canonical.
template <typename Root>
__device__ __forceinline__ void wfwd16_lazy(u64 (&x)[16], const u64* tw, const u64* tws, u64 p, Root root) {
  const u64 p2 = 2 * p;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d = 8 >> s;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u & d) continue;
      const int wi = root(s, u);
      const u64 a = x[u] >= p2 ? x[u] - p2 : x[u];
      const u64 y = mulshoup_lazy(x[u + d], tw[wi], tws[wi], p);
      x[u] = a + y;
      x[u + d] = a - y + p2;
    }
  }
}

template <typename Root>
__device__ __forceinline__ void winv16_lazy(u64 (&x)[16], const u64* tw, const u64* tws, u64 p, Root root) {
  const u64 p2 = 2 * p;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d = 1 << s;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u & d) continue;
      const int wi = root(s, u);
      const u64 a = x[u], b = x[u + d], t = a + b;
      x[u] = t >= p2 ? t - p2 : t;
      x[u + d] = mulshoup_lazy(a - b + p2, tw[wi], tws[wi], p);
    }
  }
}

__global__ __launch_bounds__(kWT) void wk_fwd_cols(const u64* src, u64* dst, long long ss,
                                                   long long ds, LimbList list, WideTables T) {
  __shared__ u64 sh[256 * kWPad];
  const int e = blockIdx.y;
  const long long g = blockIdx.z;
  const int pi = list.prime[e];
  const u64 p = T.p[pi];
  const u64* tw = T.fwd + (size_t)pi * kN;
  const u64* tws = T.fwd_s + (size_t)pi * kN;
  const u64* in = src + g * ss + (long long)list.off[e] * kN;
  u64* out = dst + g * ds + (long long)list.off[e] * kN;
  const int tid = threadIdx.x, cl = tid & 15, r = tid >> 4, c = blockIdx.x * 16 + cl;
  u64 x[16];
  // rows r + 16 u of column c: stages 0..3 (row distances 128 .. 16), root (1 << s) + (u >> (4 - s))
#pragma unroll
  for (int u = 0; u < 16; ++u) x[u] = in[c + 256 * (r + 16 * u)];
  wfwd16_lazy(x, tw, tws, p, [](int s, int u) { return (1 << s) + (u >> (4 - s)); });
#pragma unroll
  for (int u = 0; u < 16; ++u) sh[(r + 16 * u) * kWPad + cl] = x[u];
  __syncthreads();
  // rows 16 q + m (q = r): stages 4..7 (row distances 8 .. 1), root (16 << s) + ((16 q + m) >> (4 - s))
  const int q = r;
#pragma unroll
  for (int m = 0; m < 16; ++m) x[m] = sh[(16 * q + m) * kWPad + cl];
  wfwd16_lazy(x, tw, tws, p, [q](int s, int m) { return (16 << s) + ((16 * q + m) >> (4 - s)); });
#pragma unroll
  for (int m = 0; m < 16; ++m) out[c + 256 * (16 * q + m)] = wcanon4(x[m], p);
}

__global__ __launch_bounds__(kWT) void wk_fwd_rows(u64* __restrict__ dst, long long ds, LimbList list, WideTables T) {
  __shared__ u64 sh[16 * 272];
  const int e = blockIdx.y;
  const long long g = blockIdx.z;
  const int pi = list.prime[e];
  const u64 p = T.p[pi];
  const u64* tw = T.fwd + (size_t)pi * kN;
  const u64* tws = T.fwd_s + (size_t)pi * kN;
  u64* io = dst + g * ds + (long long)list.off[e] * kN + (long long)blockIdx.x * 4096;
  const int tid = threadIdx.x, rr = tid >> 4, lane = tid & 15, r = blockIdx.x * 16 + rr;
  u64* row = sh + rr * 272;
  u64 x[16];
  // elements lane + 16 u of row r: stages 8..11 (distances 128 .. 16),
  // root (256 << s) + r (1 << s) + (u >> (4 - s))
#pragma unroll
  for (int u = 0; u < 16; ++u) x[u] = io[rr * 256 + lane + 16 * u];
  wfwd16_lazy(x, tw, tws, p, [r](int s, int u) { return (256 << s) + (r << s) + (u >> (4 - s)); });
#pragma unroll
  for (int u = 0; u < 16; ++u) row[wpad(lane + 16 * u)] = x[u];
  __syncthreads();
  // elements 16 q + m (q = lane): stages 12..15 (distances 8 .. 1),
  // root (4096 << s) + r (16 << s) + ((16 q + m) >> (4 - s))
  const int q = lane;
#pragma unroll
  for (int m = 0; m < 16; ++m) x[m] = row[wpad(16 * q + m)];
  wfwd16_lazy(x, tw, tws, p, [r, q](int s, int m) { return (4096 << s) + (r << (4 + s)) + ((16 * q + m) >> (4 - s)); });
#pragma unroll
  for (int m = 0; m < 16; ++m) row[wpad(16 * q + m)] = wcanon4(x[m], p);
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 16; ++u) io[rr * 256 + lane + 16 * u] = row[wpad(lane + 16 * u)];
}

// Inverse transform (Gentleman-Sande with psi^-brv roots, then N^-1): the first eight stages act
// on the rows, the last eight on the columns, which also apply N^-1.
__global__ __launch_bounds__(kWT) void wk_inv_rows(const u64* src, u64* dst, long long ss,
                                                   long long ds, LimbList list, WideTables T) {
  __shared__ u64 sh[16 * 272];
  const int e = blockIdx.y;
  const long long g = blockIdx.z;
  const int pi = list.prime[e];
  const u64 p = T.p[pi];
  const u64* tw = T.inv + (size_t)pi * kN;
  const u64* tws = T.inv_s + (size_t)pi * kN;
  const u64* in = src + g * ss + (long long)list.off[e] * kN + (long long)blockIdx.x * 4096;
  u64* out = dst + g * ds + (long long)list.off[e] * kN + (long long)blockIdx.x * 4096;
  const int tid = threadIdx.x, rr = tid >> 4, lane = tid & 15, r = blockIdx.x * 16 + rr;
  u64* row = sh + rr * 272;
#pragma unroll
  for (int u = 0; u < 16; ++u) row[wpad(lane + 16 * u)] = in[rr * 256 + lane + 16 * u];
  __syncthreads();
  u64 x[16];
  // elements 16 q + m (q = lane): stages 0..3 (distances 1 .. 8),
  // root (32768 >> s) + r (128 >> s) + ((16 q + m) >> (s + 1))
  const int q = lane;
#pragma unroll
  for (int m = 0; m < 16; ++m) x[m] = row[wpad(16 * q + m)];
  winv16_lazy(x, tw, tws, p, [r, q](int s, int m) { return (32768 >> s) + r * (128 >> s) + ((16 * q + m) >> (s + 1)); });
#pragma unroll
  for (int m = 0; m < 16; ++m) row[wpad(16 * q + m)] = x[m];
  __syncthreads();
  // elements lane + 16 u: stages 4..7 (distances 16 .. 128), root (2048 >> s) + r (8 >> s) + (u >> (s + 1))
#pragma unroll
  for (int u = 0; u < 16; ++u) x[u] = row[wpad(lane + 16 * u)];
  winv16_lazy(x, tw, tws, p, [r](int s, int u) { return (2048 >> s) + r * (8 >> s) + (u >> (s + 1)); });
#pragma unroll
  for (int u = 0; u < 16; ++u) out[rr * 256 + lane + 16 * u] = wcanon2(x[u], p);
}

__global__ __launch_bounds__(kWT) void wk_inv_cols(u64* __restrict__ dst, long long ds, LimbList list, WideTables T) {
  __shared__ u64 sh[256 * kWPad];
  const int e = blockIdx.y;
  const long long g = blockIdx.z;
  const int pi = list.prime[e];
  const u64 p = T.p[pi];
  const u64* tw = T.inv + (size_t)pi * kN;
  const u64* tws = T.inv_s + (size_t)pi * kN;
  const u64 ni = T.ninv[pi], nis = T.ninv_s[pi];
  u64* io = dst + g * ds + (long long)list.off[e] * kN;
  const int tid = threadIdx.x, cl = tid & 15, r = tid >> 4, c = blockIdx.x * 16 + cl;
  u64 x[16];
  // rows 16 q + m of column c (q = r): stages 8..11 (row distances 1 .. 8), root (128 >> s) + ((16 q + m) >> (s + 1))
  const int q = r;
#pragma unroll
  for (int m = 0; m < 16; ++m) x[m] = io[c + 256 * (16 * q + m)];
  winv16_lazy(x, tw, tws, p, [q](int s, int m) { return (128 >> s) + ((16 * q + m) >> (s + 1)); });
#pragma unroll
  for (int m = 0; m < 16; ++m) sh[(16 * q + m) * kWPad + cl] = x[m];
  __syncthreads();
  // rows r + 16 u: stages 12..15 (row distances 16 .. 128), root (8 >> s) + (u >> (s + 1)); then N^-1
#pragma unroll
  for (int u = 0; u < 16; ++u) x[u] = sh[(r + 16 * u) * kWPad + cl];
  winv16_lazy(x, tw, tws, p, [](int s, int u) { return (8 >> s) + (u >> (s + 1)); });
#pragma unroll
  for (int u = 0; u < 16; ++u) io[c + 256 * (r + 16 * u)] = wmulc(x[u], ni, nis, p);
}

// ----------------------------------------------------------------------------- base conversion
// dst[item][slot t][k] = sum_s ybar_s * (B / b_s) mod t, ybar_s the centered representative of
// y_s = x_s (B / b_s)^-1 mod b_s (the oracle's base_conv).  Sources are the ns consecutive limbs from
// src_off.  The sum is taken lazily: with |ybar_s| < b_s / 2 < 2^60 and the constants in Montgomery
// form f = (B / b_s) 2^64 mod t (negated, t - f, for a negative ybar_s), every term is a positive
// 128-bit product and the whole sum stays below 2^63 t (ns <= 8), so one Montgomery reduction
// (x + m t) / 2^64, m = x (-t^-1) mod 2^64, lands it in [0, 2t) with the 2^64 factor removed.
// Grid (N / 256, items).
__global__ __launch_bounds__(256) void wk_conv(const u64* __restrict__ src, long long src_item, int src_off,
                                               u64* __restrict__ dst, long long dst_item,
                                               const WideConv* __restrict__ cc, WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const long long it = blockIdx.y;
  const int ns = cc->ns, nt = cc->nt;
  u64 y[kMaxAlpha];
  bool neg[kMaxAlpha];
#pragma unroll
  for (int s = 0; s < kMaxAlpha; ++s) {
    y[s] = 0;
    neg[s] = false;
    if (s < ns) {
      const u64 b = T.p[cc->src_prime[s]];
      const u64 v = wmulc(src[it * src_item + (long long)(src_off + s) * kN + k], cc->hinv[s], cc->hinv_s[s], b);
      neg[s] = 2 * v > b;
      y[s] = neg[s] ? b - v : v;
    }
  }
  for (int t = 0; t < nt; ++t) {
    const u64 q = T.p[cc->dst_prime[t]];
    u128 x = 0;
#pragma unroll
    for (int s = 0; s < kMaxAlpha; ++s) {
      if (s >= ns) break;
      const u64 f = cc->hmod_m[s][t];
      x += (u128)y[s] * (neg[s] ? q - f : f);
    }
    const u64 m = (u64)x * cc->tneg_inv[t];
    u64 r = (u64)((x + (u128)m * q) >> 64);
    r = r >= q ? r - q : r;
    dst[it * dst_item + (long long)cc->dst_slot[t] * kN + k] = r;
  }
}

// The same conversion on the int8 matrix cores.  Each source residue is centered (ybar_s, |ybar_s| <
// b_s / 2 < 2^60) and written as the 64-bit word of its eight balanced base-256 digits d_{s,a}
// (byte a = d_{s,a} + 128 of ybar_s + 0x80..80; the XOR turns each byte into d_{s,a} as int8).  With
// the digits e_{s,a,t,c} of K_{s,a,t} = (B / b_s) 256^a mod t (fill_wide_digits), one
// v_mfma_i32_16x16x64_i8 per output digit c gives C_c = sum_{s,a} d_{s,a} e_{s,a,t,c} for 16 targets x 16
// coefficients (K = 8 sources x 8 digit bytes; |C_c| <= 64 * 128^2 = 2^20), and
//   sum_c 256^c C_c = sum_{s,a} d_{s,a} K_{s,a,t} == sum_s ybar_s (B / b_s)  (mod t),
// the conversion's sum.  The fold pairs the byte positions, estimates the quotient by t in FP64
// (fold_inv = fl(1 / t)) and takes the remainder exactly in wrapping 64-bit arithmetic, then one
// correction into [0, t): the residue wk_conv returns.  Operand layout (measured): lane l supplies A row l % 16 and B column l % 16 with K bytes
// 16 (l / 16) .. +15 and receives D rows 4 (l / 16) + r, column l % 16 in register r.  Lane (q, j)
// therefore feeds sources 2q and 2q + 1 of coefficient j of its wave's tile of 16 coefficients and
// folds targets 16 G + 4q + r of that coefficient.  Grid (N / (64 TPW), items): each of the four
// waves takes TPW consecutive tiles, whose source words it requests together (the kernel is bound
// by the memory requests in flight, not by its arithmetic).
constexpr int kWmGroups = (kMaxPrimes + 15) / 16;

template <int TPW>
__global__ __launch_bounds__(256) void wk_mconv(const u64* __restrict__ src, long long src_item, int src_off,
                                                u64* __restrict__ dst, long long dst_item,
                                                const WideConv* __restrict__ cc, const wv4i* __restrict__ dig,
                                                WideTables T) {
  __shared__ wv4i A[kWmGroups * 8 * 64];
  const int ns = cc->ns, nt = cc->nt, groups = (nt + 15) >> 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, j = lane & 15;
  const long long it = blockIdx.y;
  const int tile0 = (blockIdx.x * 4 + wave) * TPW;
  // every source word of the wave's tiles is requested before anything waits on memory
  u64 raw[TPW][2], b[2], hv[2], hs[2];
  bool act[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int sidx = 2 * q + h;
    act[h] = sidx < ns;
    const int si = act[h] ? sidx : 0;
    const u64* sp = src + it * src_item + (long long)(src_off + si) * kN;
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) raw[tt][h] = act[h] ? sp[(tile0 + tt) * 16 + j] : 0;
    b[h] = T.p[cc->src_prime[si]];
    hv[h] = cc->hinv[si];
    hs[h] = cc->hinv_s[si];
  }
  const wv4i* __restrict__ tab = dig + cc->dig_off;
  for (int i = threadIdx.x; i < groups * 512; i += 256) A[i] = tab[i];
  __syncthreads();
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int k = (tile0 + tt) * 16 + j;
    u64 w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      w[h] = 0;
      if (act[h]) {
        w[h] = wdigits(wmulc(raw[tt][h], hv[h], hs[h], b[h]), b[h]);
      }
    }
    const wv4i bv = {(int)(uint32_t)w[0], (int)(uint32_t)(w[0] >> 32), (int)(uint32_t)w[1], (int)(uint32_t)(w[1] >> 32)};
    for (int G = 0; G < groups; ++G) {
      wv4i acc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
        acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[(G * 8 + c) * 64 + lane], bv, wv4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * G + 4 * q + r;
        if (t < nt)
          dst[it * dst_item + (long long)cc->dst_slot[t] * kN + k] = wfold(acc, r, T.p[cc->dst_prime[t]], cc->fold_inv[t]);
      }
    }
  }
}

// The centered lift of one coefficient-domain limb (prime src_pi) to limbs first .. first + gridDim.y - 1
// (limb i modulo prime i).  Grid (N / 256, targets, items).
__global__ __launch_bounds__(256) void wk_lift(const u64* __restrict__ src, long long src_item, int src_pi,
                                               u64* __restrict__ dst, long long dst_item, int first, WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = first + blockIdx.y;
  const long long it = blockIdx.z;
  const u64 ql = T.p[src_pi];
  const Barrett64 br = wbar(T, i);
  const u64 v = src[it * src_item + k];
  u64 r;
  if (2 * v > ql) {
    const u64 m = barrett_reduce((u128)(ql - v), br);
    r = m ? br.p - m : 0;
  } else {
    r = barrett_reduce((u128)v, br);
  }
  dst[it * dst_item + (long long)i * kN + k] = r;
}

// --------------------------------------------------------------------------------- key switch parts
struct WKeys {
  const u64* k[kWideChunk];
};
struct WGal {
  uint32_t g[kWideChunk];
};

__device__ __forceinline__ uint32_t wbrv16(uint32_t x) { return __brev(x) >> 16; }

// sigma_g of every limb of item it with g = G.g[it] (NTT domain).  Grid (N / 256, limbs, items).
__global__ __launch_bounds__(256) void wk_automorph(const u64* __restrict__ in, long long in_item,
                                                    u64* __restrict__ out, long long out_item, WGal G) {
  const uint32_t k = blockIdx.x * 256 + threadIdx.x;
  const long long it = blockIdx.z, limb = blockIdx.y;
  const uint32_t e = ((2u * wbrv16(k) + 1u) * G.g[it]) & (2u * kN - 1u);
  const uint32_t src = wbrv16((e - 1u) >> 1);
  out[it * out_item + limb * kN + k] = in[it * in_item + limb * kN + src];
}

// The inner product fused with the forward NTT's row pass: for every digit j, the block takes the
// column-pass output of digit j on its 16 rows of limb e (the digit's own limb: the NTT-domain input
// d as it is), finishes the transform in registers (the wk_fwd_rows body), and multiplies by both
// key halves, accumulating over the digits on chip; acc[item][comp][e] is written once.
// Grid (16, ell + K, items).
__global__ __launch_bounds__(kWT) void wk_ks_ip_rows(const u64* __restrict__ ext, long long ext_item,
                                                     const u64* __restrict__ d, long long d_item, int alpha,
                                                     int beta, WKeys keys, int ell, int L, int K, int beta_max,
                                                     u64* __restrict__ acc, long long acc_item, WideTables T) {
  __shared__ u64 sh[16 * 272];
  const int e = blockIdx.y;
  const long long it = blockIdx.z;
  const int ext_l = ell + K;
  const int pi = e < ell ? e : L + (e - ell);
  const u64 p = T.p[pi];
  const Barrett64 br = wbar(T, pi);
  const u64* tw = T.fwd + (size_t)pi * kN;
  const u64* tws = T.fwd_s + (size_t)pi * kN;
  const int tid = threadIdx.x, rr = tid >> 4, lane = tid & 15, r = blockIdx.x * 16 + rr;
  const long long base = (long long)blockIdx.x * 4096 + rr * 256 + lane;  // element lane + 16 u of row r
  const u64* key = keys.k[it];
  const long long comp = (long long)beta_max * (L + K) * kN;
  const int own = e < ell ? e / alpha : -1;
  u64* row = sh + rr * 272;
  u64 ab[16], aa[16], x[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) ab[u] = aa[u] = 0;
  for (int j = 0; j < beta; ++j) {
    if (j == own) {
      const u64* src = d + it * d_item + (long long)e * kN + base;
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = src[16 * u];
    } else {
      const u64* src = ext + it * ext_item + ((long long)j * ext_l + e) * kN + base;
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = src[16 * u];
      wfwd16(x, tw, tws, p, [r](int s, int u) { return (256 << s) + (r << s) + (u >> (4 - s)); });
#pragma unroll
      for (int u = 0; u < 16; ++u) row[wpad(lane + 16 * u)] = x[u];
      __syncthreads();
      const int q = lane;
#pragma unroll
      for (int m = 0; m < 16; ++m) x[m] = row[wpad(16 * q + m)];
      wfwd16(x, tw, tws, p,
             [r, q](int s, int m) { return (4096 << s) + (r << (4 + s)) + ((16 * q + m) >> (4 - s)); });
#pragma unroll
      for (int m = 0; m < 16; ++m) row[wpad(16 * q + m)] = x[m];
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = row[wpad(lane + 16 * u)];
      __syncthreads();  // the LDS rows are rewritten by the next digit
    }
    const u64* kb = key + ((long long)j * (L + K) + pi) * kN + base;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      ab[u] = wadd(ab[u], mulmod64(x[u], kb[16 * u], br), p);
      aa[u] = wadd(aa[u], mulmod64(x[u], kb[comp + 16 * u], br), p);
    }
  }
  u64* o = acc + it * acc_item + (long long)e * kN + base;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    o[16 * u] = ab[u];
    o[(long long)ext_l * kN + 16 * u] = aa[u];
  }
}

// out[i] = (x[i] - cv[i]) P^-1 mod q_i (+ add1[i]) (+ add2[i]).  Grid (N / 256, ell, items).
__global__ __launch_bounds__(256) void wk_ks_out(const u64* x, long long x_item, const u64* __restrict__ cv,
                                                 long long cv_item, const u64* add1, long long add1_item,
                                                 const u64* add2, long long add2_item, u64* out, long long out_item,
                                                 const u64* __restrict__ fac, const u64* __restrict__ fac_s,
                                                 WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long it = blockIdx.z;
  const u64 q = T.p[i];
  const long long o = (long long)i * kN + k;
  u64 v = wmulc(wsub(x[it * x_item + o], cv[it * cv_item + o], q), fac[i], fac_s[i], q);
  if (add1) v = wadd(v, add1[it * add1_item + o], q);
  if (add2) v = wadd(v, add2[it * add2_item + o], q);
  out[it * out_item + o] = v;
}

// Extended-basis output: out[e] = acc[e] (+ P * s0[e] on the Q limbs) (+ add[e]).  Grid (N / 256, ell + K, items).
__global__ __launch_bounds__(256) void wk_ks_ext_out(const u64* __restrict__ acc, long long acc_item,
                                                     const u64* __restrict__ s0, long long s0_item, const u64* add,
                                                     long long add_item, u64* out, long long out_item, int ell, int L,
                                                     WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int e = blockIdx.y;
  const long long it = blockIdx.z;
  const int pi = e < ell ? e : L + (e - ell);
  const u64 q = T.p[pi];
  const long long o = (long long)e * kN + k;
  u64 v = acc[it * acc_item + o];
  if (s0 && e < ell) v = wadd(v, wmulc(s0[it * s0_item + o], T.pmod[pi], T.pmod_s[pi], q), q);
  if (add) v = wadd(v, add[it * add_item + o], q);
  out[it * out_item + o] = v;
}

// Hoisted rotations.  Item it of a launch is input (first + it) % inputs rotated by G.g[it]; its
// extended digits (the ModUp of c1, NTT domain, [inputs][beta][ell + K][N], the digit's own limbs
// included) are read through sigma_g, which commutes with ModUp (the centered lift is odd-symmetric):
// acc[item][comp][e] = sum_j sigma(digit_j)[e] * key_j[comp][prime(e)].  Grid (N / 256, ell + K, items).
__global__ __launch_bounds__(256) void wk_ks_ip_h(const u64* __restrict__ digits, int inputs, int first, WGal G,
                                                  WKeys keys, int beta, int ell, int L, int K, int beta_max,
                                                  u64* __restrict__ acc, long long acc_item, WideTables T) {
  const uint32_t k = blockIdx.x * 256 + threadIdx.x;
  const int e = blockIdx.y;
  const long long it = blockIdx.z;
  const int ext_l = ell + K;
  const long long in = (first + it) % inputs;
  const uint32_t g = G.g[it];
  const uint32_t ex = ((2u * wbrv16(k) + 1u) * g) & (2u * kN - 1u);
  const uint32_t src = wbrv16((ex - 1u) >> 1);
  const int pi = e < ell ? e : L + (e - ell);
  const u64 p = T.p[pi], p2 = 2 * p, mneg = T.mneg[pi];
  const u64* key = keys.k[it];
  const long long comp = (long long)beta_max * (L + K) * kN;
  const u64* dg = digits + (in * beta * ext_l + e) * (long long)kN + src;
  u64 ab = 0, aa = 0;  // Montgomery products summed below 2p, then one product by 2^64 mod p
  for (int j = 0; j < beta; ++j) {
    const u64 x = dg[(long long)j * ext_l * kN];
    const long long ko = ((long long)j * (L + K) + pi) * kN + k;
    const u64 vb = ab + wmont(x, key[ko], p, mneg), va = aa + wmont(x, key[comp + ko], p, mneg);
    ab = vb >= p2 ? vb - p2 : vb;
    aa = va >= p2 ? va - p2 : va;
  }
  u64* o = acc + it * acc_item + (long long)e * kN + k;
  o[0] = wmulc(ab, T.r64[pi], T.r64_s[pi], p);
  o[(long long)ext_l * kN] = wmulc(aa, T.r64[pi], T.r64_s[pi], p);
}

// sigma of every limb of input (first + it) % inputs by G.g[it].  Grid (N / 256, limbs, items).
__global__ __launch_bounds__(256) void wk_automorph_h(const u64* __restrict__ in, long long in_item, int inputs,
                                                      int first, u64* __restrict__ out, long long out_item, WGal G) {
  const uint32_t k = blockIdx.x * 256 + threadIdx.x;
  const long long it = blockIdx.z, limb = blockIdx.y;
  const long long src_item = (first + it) % inputs;
  const uint32_t e = ((2u * wbrv16(k) + 1u) * G.g[it]) & (2u * kN - 1u);
  const uint32_t src = wbrv16((e - 1u) >> 1);
  out[it * out_item + limb * kN + k] = in[src_item * in_item + limb * kN + src];
}

// ------------------------------------------------------------------------------------ elementwise
struct WPrimeMap {
  uint8_t prime[kMaxPrimes];
};
struct WScalars {
  u64 s[kMaxPrimes];
  u64 ss[kMaxPrimes];
};

template <int OP>
__global__ __launch_bounds__(256) void wk_poly_op(u64* out, const u64* a, const u64* b, long long out_stride,
                                                  long long a_stride, long long b_stride, WPrimeMap pm, WScalars sc,
                                                  WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int limb = blockIdx.y;
  const int pi = pm.prime[limb];
  const u64 p = T.p[pi];
  const long long lo = (long long)limb * kN + k;
  const long long z = blockIdx.z;
  const u64 x = a[z * a_stride + lo];
  u64 r;
  if constexpr (OP == HCK_OP_ADD) {
    r = wadd(x, b[z * b_stride + lo], p);
  } else if constexpr (OP == HCK_OP_SUB) {
    r = wsub(x, b[z * b_stride + lo], p);
  } else if constexpr (OP == HCK_OP_NEG) {
    r = x ? p - x : 0;
  } else if constexpr (OP == HCK_OP_MUL) {
    r = mulmod64(x, b[z * b_stride + lo], wbar(T, pi));
  } else if constexpr (OP == HCK_OP_MAC) {
    r = wadd(out[z * out_stride + lo], mulmod64(x, b[z * b_stride + lo], wbar(T, pi)), p);
  } else if constexpr (OP == HCK_OP_MUL_SCALAR) {
    r = wmulc(x, sc.s[limb], sc.ss[limb], p);
  } else if constexpr (OP == HCK_OP_ADD_SCALAR) {
    r = wadd(x, sc.s[limb], p);
  } else {  // HCK_OP_MUL_XHALF: zeta4 on the slots k < N/2, -zeta4 above
    const u64 m = wmulc(x, T.zeta4[pi], T.zeta4_s[pi], p);
    r = k < kN / 2 ? m : (m ? p - m : 0);
  }
  out[z * out_stride + lo] = r;
}

__global__ __launch_bounds__(256) void wk_tensor(const u64* __restrict__ a0, const u64* __restrict__ a1, long long as,
                                                 const u64* __restrict__ b0, const u64* __restrict__ b1, long long bs,
                                                 u64* __restrict__ d0, u64* __restrict__ d1, u64* __restrict__ d2,
                                                 long long dst, int d01_from, WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long z = blockIdx.z;
  const Barrett64 br = wbar(T, i);
  const long long lo = (long long)i * kN + k;
  const u64 x1 = a1[z * as + lo], y1 = b1[z * bs + lo];
  d2[z * dst + lo] = mulmod64(x1, y1, br);
  if (i < d01_from) return;  // d0 / d1 only on limbs d01_from.. (uniform over the block)
  const u64 x0 = a0[z * as + lo], y0 = b0[z * bs + lo];
  d0[z * dst + lo] = mulmod64(x0, y0, br);
  d1[z * dst + lo] = wadd(mulmod64(x0, y1, br), mulmod64(x1, y0, br), br.p);
}

__global__ __launch_bounds__(256) void wk_weighted_sum(const u64* __restrict__ in, long long in_stride, int n,
                                                       const u64* __restrict__ w, u64* __restrict__ out,
                                                       long long out_stride, int limbs, WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long g = blockIdx.z;
  const Barrett64 br = wbar(T, i);
  const u64* wg = w + g * (long long)n * limbs + i;
  const u64* x = in + (long long)i * kN + k;
  u64 acc = 0;
  for (int j = 0; j < n; ++j) acc = wadd(acc, mulmod64(x[(long long)j * in_stride], wg[(long long)j * limbs], br), br.p);
  out[g * out_stride + (long long)i * kN + k] = acc;
}

constexpr int kWLcMaxPtrs = 256;
constexpr int kWLcMaxGroups = 64;
struct WLcPtrs {
  const u64* x[kWLcMaxPtrs];
  u64* out[kWLcMaxGroups];
};

__global__ __launch_bounds__(256) void wk_lincomb(const WLcPtrs P, int terms, const u64* __restrict__ w, int limbs,
                                                  WideTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y, g = blockIdx.z;
  const Barrett64 br = wbar(T, i);
  const long long off = (long long)i * kN + k;
  u64 acc = 0;
  for (int t = 0; t < terms; ++t) {
    const u64 x = P.x[g * terms + t][off];
    acc = wadd(acc, w ? mulmod64(x, w[(long long)t * limbs + i], br) : x, br.p);
  }
  P.out[g][off] = acc;
}

constexpr int kWMaxBabies = 64;
struct WMac {
  const u64* c0[kWMaxBabies];
  const u64* c1[kWMaxBabies];
};

// res[c][g][i][l][k] = sum_b pts[g B + b][l][k] * baby_b[c][i][l][k] (mod q_l), the FP64 MAC's tiling
// (bsgs.hip: k_bsgs_mac): a thread owns one coefficient of one limb and a kWTI x kWTG tile of (input,
// giant) accumulators for both components; per baby step it reads kWTG plaintext words and 2 kWTI baby
// words for 2 kWTI kWTG products (the next step's words are in flight while the current one computes).
// The products of canonical operands (below p^2) are summed exactly in 128 bits; every kFoldEvery baby
// steps (kFoldEvery p^2 < p 2^64 for p < 2^61) a sum is folded back to its canonical residue by one
// Montgomery reduction and one product with 2^64 mod p, and the last fold gives the result.  All tiles
// of one (limb, 128-coefficient) unit are dealt to one XCD, so the unit's plaintext and baby words come
// from HBM once.
constexpr int kWMacThreads = 128;
constexpr int kWTI = 4;
constexpr int kWTG = 4;
constexpr int kFoldEvery = 8;

struct WMacOps {
  u64 w[kWTG], x0[kWTI], x1[kWTI];
};

__device__ __forceinline__ void wmac_load(WMacOps& o, const WMac& P, int b, int babies, int G, int ni, int g0,
                                          int i0, const u64* __restrict__ pts, long long pt_stride,
                                          long long baby_stride, long long ln) {
#pragma unroll
  for (int g = 0; g < kWTG; ++g) {
    const int gg = g0 + g < G ? g0 + g : g0;  // clamped rows are computed but never stored
    o.w[g] = pts[((long long)gg * babies + b) * pt_stride + ln];
  }
#pragma unroll
  for (int t = 0; t < kWTI; ++t) {
    const int ii = i0 + t < ni ? i0 + t : i0;
    o.x0[t] = P.c0[b][(long long)ii * baby_stride + ln];
    o.x1[t] = P.c1[b][(long long)ii * baby_stride + ln];
  }
}


__global__ __launch_bounds__(kWMacThreads) void wk_bsgs_mac(const WMac P, long long baby_stride,
                                                            const u64* __restrict__ pts, long long pt_stride,
                                                            u64* __restrict__ res, int inputs, int babies, int giants,
                                                            int limbs, WPrimeMap pm, int units_per_limb, int tiles_i,
                                                            int tiles_g, int total_units, WideTables T) {
  const int tiles = tiles_i * tiles_g;
  const int lin = blockIdx.x;
  const int xcd = lin % kXcds, q = lin / kXcds;
  const int unit = (q / tiles) * kXcds + xcd;
  const int tile = q % tiles;
  if (unit >= total_units) return;
  const int l = unit / units_per_limb;
  const int n = (unit % units_per_limb) * kWMacThreads + threadIdx.x;
  const int i0 = (tile % tiles_i) * kWTI, g0 = (tile / tiles_i) * kWTG;
  const int pi = pm.prime[l];
  const u64 p = T.p[pi], mneg = T.mneg[pi], r = T.r64[pi], rs = T.r64_s[pi];
  const long long ln = (long long)l * kN + n;
  u128 acc[kWTI][2][kWTG];
#pragma unroll
  for (int t = 0; t < kWTI; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kWTG; ++g) acc[t][c][g] = 0;
  // one baby step's products; every kFoldEvery steps the sums are folded
  auto step = [&](const WMacOps& cur, int b) {
#pragma unroll
    for (int t = 0; t < kWTI; ++t)
#pragma unroll
      for (int g = 0; g < kWTG; ++g) {
        acc[t][0][g] += (u128)cur.x0[t] * cur.w[g];
        acc[t][1][g] += (u128)cur.x1[t] * cur.w[g];
      }
    if (b % kFoldEvery == kFoldEvery - 1 && b + 1 < babies) {  // the folded residue restarts the sum
#pragma unroll
      for (int t = 0; t < kWTI; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int g = 0; g < kWTG; ++g) acc[t][c][g] = wfold128(acc[t][c][g], p, mneg, r, rs);
    }
  };
  // two-stage software pipeline on two register sets: step b + 1's words load into one set while step
  // b computes from the other (the last pair reloads its own words, unused); the memory clobber and
  // the scheduling barrier keep each set's loads ahead of the products they overlap, so a step waits
  // only for its own loads
  WMacOps o0, o1;
  wmac_load(o0, P, 0, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride, ln);
  int b = 0;
  for (; b + 1 < babies; b += 2) {
    wmac_load(o1, P, b + 1, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride, ln);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o0, b);
    wmac_load(o0, P, b + 2 < babies ? b + 2 : b + 1, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride, ln);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o1, b + 1);
  }
  if (b < babies) step(o0, b);  // odd count: the last step's words are in o0
  const long long is = (long long)limbs * kN, gs = (long long)inputs * is, cs = (long long)giants * gs;
#pragma unroll
  for (int t = 0; t < kWTI; ++t) {
    if (i0 + t >= inputs) break;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kWTG; ++g)
        if (g0 + g < giants)
          res[c * cs + (long long)(g0 + g) * gs + (long long)(i0 + t) * is + ln] =
              wfold128(acc[t][c][g], p, mneg, r, rs);
  }
}

// The MAC on contexts whose primes all lie below 2^60: each canonical word is split into 30-bit halves
// (x = x1 2^30 + x0), and a product's three partial products go into three 64-bit sums without carries,
//   S0 += x0 w0,   S1 += x0 w1 + x1 w0,   S2 += x1 w1   (each partial product below 2^60, the middle pair
// below 2^61), so a product costs four 32 x 32 -> 64 multiply-adds.  Every kSFold baby steps the sums are
// normalised: the bits of S0 above 2^30 move into S1, those of S1 into S2, and S2 2^60 comes back as
// one Shoup product by 2^60 mod p (below 2p) added to S0; the invariant S0 < 2^30 + 2p, S1 < 2^30,
// S2 = 0 keeps kSFold more steps inside 64 bits (2^30 + 2^61 + 7 2^60 and 2^30 + 7 2^61 + 2^34 below
// 2^64).  The result is the canonical residue of S0 + S1 2^30 (below 2^62), the value sum_b x_b w_b
// mod p exactly, as the 128-bit MAC gives it.  Tiles of kSTI inputs x kSTG giants per thread.
constexpr int kSTI = 2;
constexpr int kSTG = 4;
constexpr int kSFold = 7;
constexpr u64 kM30 = (1ULL << 30) - 1;

struct WSplitOps {
  u64 w[kSTG], x0[kSTI], x1[kSTI];
};

__device__ __forceinline__ void wmac30_load(WSplitOps& o, const WMac& P, int b, int babies, int G, int ni, int g0,
                                            int i0, const u64* __restrict__ pts, long long pt_stride,
                                            long long baby_stride, long long ln) {
#pragma unroll
  for (int g = 0; g < kSTG; ++g) {
    const int gg = g0 + g < G ? g0 + g : g0;  // clamped rows are computed but never stored
    o.w[g] = pts[((long long)gg * babies + b) * pt_stride + ln];
  }
#pragma unroll
  for (int t = 0; t < kSTI; ++t) {
    const int ii = i0 + t < ni ? i0 + t : i0;
    o.x0[t] = P.c0[b][(long long)ii * baby_stride + ln];
    o.x1[t] = P.c1[b][(long long)ii * baby_stride + ln];
  }
}

__global__ __launch_bounds__(kWMacThreads) void wk_bsgs_mac30(const WMac P, long long baby_stride,
                                                              const u64* __restrict__ pts, long long pt_stride,
                                                              u64* __restrict__ res, int inputs, int babies,
                                                              int giants, int limbs, WPrimeMap pm, int units_per_limb,
                                                              int tiles_i, int tiles_g, int total_units, WideTables T) {
  const int tiles = tiles_i * tiles_g;
  const int lin = blockIdx.x;
  const int xcd = lin % kXcds, q = lin / kXcds;
  const int unit = (q / tiles) * kXcds + xcd;
  const int tile = q % tiles;
  if (unit >= total_units) return;
  const int l = unit / units_per_limb;
  const int n = (unit % units_per_limb) * kWMacThreads + threadIdx.x;
  const int i0 = (tile % tiles_i) * kSTI, g0 = (tile / tiles_i) * kSTG;
  const int pi = pm.prime[l];
  const u64 p = T.p[pi], c60 = T.r60[pi], c60s = T.r60_s[pi];
  const long long ln = (long long)l * kN + n;
  u64 s0[kSTI][2][kSTG], s1[kSTI][2][kSTG], s2[kSTI][2][kSTG];
#pragma unroll
  for (int t = 0; t < kSTI; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kSTG; ++g) s0[t][c][g] = s1[t][c][g] = s2[t][c][g] = 0;
  auto step = [&](const WSplitOps& o, int b) {
    uint32_t wl[kSTG], wh[kSTG];
#pragma unroll
    for (int g = 0; g < kSTG; ++g) {
      wl[g] = (uint32_t)o.w[g] & (uint32_t)kM30;
      wh[g] = (uint32_t)(o.w[g] >> 30);
    }
#pragma unroll
    for (int t = 0; t < kSTI; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u64 x = c ? o.x1[t] : o.x0[t];
        const uint32_t xl = (uint32_t)x & (uint32_t)kM30, xh = (uint32_t)(x >> 30);
#pragma unroll
        for (int g = 0; g < kSTG; ++g) {
          s0[t][c][g] += (u64)xl * wl[g];
          s1[t][c][g] += (u64)xl * wh[g];
          s1[t][c][g] += (u64)xh * wl[g];
          s2[t][c][g] += (u64)xh * wh[g];
        }
      }
    if (b % kSFold == kSFold - 1 && b + 1 < babies) {  // uniform
#pragma unroll
      for (int t = 0; t < kSTI; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int g = 0; g < kSTG; ++g) {
            u64 a = s0[t][c][g], m = s1[t][c][g], h = s2[t][c][g];
            m += a >> 30;
            a &= kM30;
            h += m >> 30;
            m &= kM30;
            s0[t][c][g] = a + mulshoup_lazy(h, c60, c60s, p);
            s1[t][c][g] = m;
            s2[t][c][g] = 0;
          }
    }
  };
  // the two-register-set pipeline of wk_bsgs_mac
  WSplitOps o0, o1;
  wmac30_load(o0, P, 0, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride, ln);
  int b = 0;
  for (; b + 1 < babies; b += 2) {
    wmac30_load(o1, P, b + 1, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride, ln);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o0, b);
    wmac30_load(o0, P, b + 2 < babies ? b + 2 : b + 1, babies, giants, inputs, g0, i0, pts, pt_stride, baby_stride,
                ln);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o1, b + 1);
  }
  if (b < babies) step(o0, b);
  const u64 mneg = T.mneg[pi], r = T.r64[pi], rs = T.r64_s[pi];
  const long long is = (long long)limbs * kN, gs = (long long)inputs * is, cs = (long long)giants * gs;
#pragma unroll
  for (int t = 0; t < kSTI; ++t) {
    if (i0 + t >= inputs) break;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kSTG; ++g)
        if (g0 + g < giants) {
          // the last block's sums, normalised as above, then S0 + S1 2^30 + S2 2^60 reduced exactly
          u64 a = s0[t][c][g], m = s1[t][c][g], h = s2[t][c][g];
          m += a >> 30;
          a &= kM30;
          h += m >> 30;
          m &= kM30;
          const u64 v = a + (m << 30) + mulshoup_lazy(h, c60, c60s, p);  // below 2^61 + 2^30
          res[c * cs + (long long)(g0 + g) * gs + (long long)(i0 + t) * is + ln] = wfold128((u128)v, p, mneg, r, rs);
        }
  }
}

// ---------------------------------------------------------------------------------------- encode
constexpr double kWideEncodeCap = 2305843009213693952.0;  // 2^61, as the FP64 path

// The rounding of the special IFFT's output (the FP64 path's expression, contraction off) fused with
// the forward transform's column pass: the block rounds the 16 columns' 4096 coefficients once, then
// for each of its listed limbs reduces them modulo the limb's prime and runs the column stages (as
// wk_fwd_cols); wk_fwd_rows finishes the transform.  Grid (16, limb chunks of lpb, rows).
__global__ __launch_bounds__(kWT) void wk_encode_cols(const double* __restrict__ vre, const double* __restrict__ vim,
                                                      double scale, u64* __restrict__ out, long long out_stride,
                                                      LimbList list, int lpb, int* __restrict__ overflow,
                                                      WideTables T) {
  __shared__ u64 sh[256 * kWPad];
  const long long row = blockIdx.z;
  const int tid = threadIdx.x, cl = tid & 15, r = tid >> 4, c = blockIdx.x * 16 + cl;
  const double* re = vre + row * (kN / 2);
  const double* im = vim + row * (kN / 2);
  u64 mag[16];
  unsigned neg = 0;
  bool big = false;
  {
#pragma clang fp contract(off)
    const double inv_n = 1.0 / (double)(kN / 2);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int n = c + 256 * (r + 16 * u);
      const int h = n >= kN / 2;
      const int slot = (int)(__brev((unsigned)(n - h * (kN / 2))) >> (32 - (kLogN - 1)));
      const double w = (h ? im : re)[slot] * inv_n;
      const double a = round_away(w * scale);
      const bool b = !(fabs(a) < kWideEncodeCap);
      big |= b;
      mag[u] = b ? 0 : (u64)fabs(a);
      neg |= (a < 0 ? 1u : 0u) << u;
    }
  }
  if (big) overflow[row] = 1;
  u64* d = out + row * out_stride;
  const int e_end = min(list.n, ((int)blockIdx.y + 1) * lpb);  // this block: limbs [blockIdx.y lpb, e_end)
  for (int e = (int)blockIdx.y * lpb; e < e_end; ++e) {
    const int pi = list.prime[e];
    const Barrett64 br = wbar(T, pi);
    const u64 p = br.p;
    const u64* tw = T.fwd + (size_t)pi * kN;
    const u64* tws = T.fwd_s + (size_t)pi * kN;
    u64 x[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const u64 v = barrett_reduce((u128)mag[u], br);
      x[u] = ((neg >> u) & 1u) && v ? p - v : v;
    }
    wfwd16_lazy(x, tw, tws, p, [](int s, int u) { return (1 << s) + (u >> (4 - s)); });
#pragma unroll
    for (int u = 0; u < 16; ++u) sh[(r + 16 * u) * kWPad + cl] = x[u];
    __syncthreads();
    const int q = r;
#pragma unroll
    for (int m = 0; m < 16; ++m) x[m] = sh[(16 * q + m) * kWPad + cl];
    wfwd16_lazy(x, tw, tws, p, [q](int s, int m) { return (16 << s) + ((16 * q + m) >> (4 - s)); });
    u64* o = d + (long long)list.off[e] * kN;
#pragma unroll
    for (int m = 0; m < 16; ++m) o[c + 256 * (16 * q + m)] = wcanon4(x[m], p);
    __syncthreads();  // every thread has read sh before the next limb writes it
  }
}

// ------------------------------------------------------------------- the encode sidecar's stage 2
// Rows of the special IFFT's output as interleaved doubles (slot j: Re at 2 j, Im at 2 j + 1);
// coefficient n < N/2 is Re of slot n, n >= N/2 is Im of slot n - N/2 (bench/cmp/kernels/
// holmes_encode.cu:108-111), times sf, rounded half away from zero, reduced exactly by each limb's
// prime, then the forward NTT's column pass with the caller's root table (psi^brv(k) and Shoup
// companions, limb e at e * N).  A coefficient of magnitude 2^63 or more encodes as 0.  Grid
// (16, limbs, rows): 16 columns of one limb of one row per block; wk_fwd_rows finishes the NTT.
__global__ __launch_bounds__(kWT) void wk_stage2_cols(const double* __restrict__ in, long long in_stride, double sf,
                                                      u64* __restrict__ out, int limbs, const u64* __restrict__ primes,
                                                      const u64* __restrict__ roots, const u64* __restrict__ roots_s) {
  __shared__ u64 sh[256 * 16];
  const int e = blockIdx.y;
  const long long row = blockIdx.z;
  const u64 p = primes[e];
  const u64* tw = roots + (size_t)e * kN;
  const u64* tws = roots_s + (size_t)e * kN;
  const double* src = in + row * in_stride;
  u64* o = out + (row * limbs + e) * (long long)kN;
  const int tid = threadIdx.x, cl = tid & 15, r = tid >> 4, c = blockIdx.x * 16 + cl;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int k = r + 16 * m;
    const int n = c + 256 * k;
    const double v = src[n < kN / 2 ? 2 * n : 2 * (n - kN / 2) + 1];
    double a;
    {
#pragma clang fp contract(off)
      a = round_away(v * sf);
    }
    const u64 mag = fabs(a) < 9223372036854775808.0 ? (u64)fabs(a) % p : 0;
    sh[k * 16 + cl] = (a < 0 && mag) ? p - mag : mag;
  }
  __syncthreads();
  for (int st = 0; st < 8; ++st) {
    const int m = 1 << st, t = 128 >> st;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int b = r + 16 * u;
      const int k1 = (b / t) * 2 * t + (b % t), k2 = k1 + t;
      const int wi = m + b / t;
      const u64 x = sh[k1 * 16 + cl];
      const u64 y = wmulc(sh[k2 * 16 + cl], tw[wi], tws[wi], p);
      sh[k1 * 16 + cl] = wadd(x, y, p);
      sh[k2 * 16 + cl] = wsub(x, y, p);
    }
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int k = r + 16 * m;
    o[c + 256 * k] = sh[k * 16 + cl];
  }
}

}  // namespace

int encode_stage2(uint64_t* out, const double* in, long long in_stride, int rows, double sf, int limbs,
                  const uint64_t* primes, const uint64_t* roots, const uint64_t* roots_shoup, int rows_per_launch,
                  int parts, hipStream_t s) {
  if (rows <= 0 || limbs <= 0) return HCK_OK;
  if (!out || !in || !primes || !roots || !roots_shoup || limbs > kMaxList) return HCK_ERR_ARG;
  if (rows > 1 && in_stride < kN) return HCK_ERR_ARG;
  // the row pass reads the caller's tables through the wide kernels' table view
  WideTables T{};
  T.p = primes;
  T.fwd = roots;
  T.fwd_s = roots_shoup;
  LimbList list;
  list.n = limbs;
  for (int e = 0; e < limbs; ++e) {
    list.off[e] = (uint16_t)e;
    list.prime[e] = (uint8_t)e;
  }
  const int step = rows_per_launch > 0 && rows_per_launch < 65535 ? rows_per_launch : 65535;
  for (int r0 = 0; r0 < rows; r0 += step) {
    const int nr = rows - r0 < step ? rows - r0 : step;
    u64* o = out + (long long)r0 * limbs * kN;
    if (parts & 1)
      wk_stage2_cols<<<dim3(16, limbs, nr), kWT, 0, s>>>(in + (long long)r0 * in_stride, in_stride, sf, o, limbs,
                                                         primes, roots, roots_shoup);
    if (parts & 2) wk_fwd_rows<<<dim3(16, limbs, nr), kWT, 0, s>>>(o, (long long)limbs * kN, list, T);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

// ======================================================================================= set-up
u64 primitive_root_2n(u64 q, int log_n);  // context.hip: the root choice every table shares

// Balanced base-256 digits of 0 <= v < 2^62: v = sum_c e_c 256^c with every e_c in [-128, 127].
void balanced_digits(u64 v, int8_t (&e)[8]) {
  long long x = (long long)v;
  for (int c = 0; c < 8; ++c) {
    int d = (int)(x & 255);
    if (d >= 128) d -= 256;
    e[c] = (int8_t)d;
    x = (x - d) / 256;  // exact: x - d is a multiple of 256
  }
}

// The matrix-core operands of one conversion (wk_mconv): for target group G (targets 16 G .. 16 G + 15),
// output digit c and lane l, the 16 bytes lane l supplies as the A operand of
// v_mfma_i32_16x16x64_i8 -- row l % 16 (target 16 G + l % 16), K bytes 16 (l / 16) .. +15, i.e.
// source s = 2 (l / 16) + m / 8 and digit position a = m % 8 for byte m: digit c of
// K_{s,a,t} = (B / b_s) 256^a mod t (zero for t >= nt or s >= ns).  Also sets fold_inv.
void fill_wide_digits(WideConv& cc, const std::vector<u64>& P, std::vector<int8_t>& tab) {
  const int groups = (cc.nt + 15) / 16;
  cc.dig_off = (long long)(tab.size() / 16);
  const size_t base = tab.size();
  tab.resize(base + (size_t)groups * 8 * 64 * 16, 0);
  for (int t = 0; t < cc.nt; ++t) {
    const u64 qt = P[cc.dst_prime[t]];
    cc.fold_inv[t] = 1.0 / (double)qt;
    const int G = t / 16, i = t % 16;
    for (int sidx = 0; sidx < cc.ns; ++sidx) {
      u64 k = cc.hmod[sidx][t];
      for (int a = 0; a < 8; ++a) {
        int8_t e[8];
        balanced_digits(k, e);
        const int qd = sidx / 2, m = 8 * (sidx % 2) + a, l = 16 * qd + i;
        for (int c = 0; c < 8; ++c) tab[base + (((size_t)G * 8 + c) * 64 + l) * 16 + m] = e[c];
        k = hmul(k, 256 % qt, qt);
      }
    }
  }
}

int wide_init(hck_context* c) {
  const int L = c->L, K = c->K, alpha = c->alpha, bmax = c->beta_max;
  const size_t np = (size_t)c->np, n = kN;
  const std::vector<u64>& P = c->primes;
  std::vector<u64> p(np), mu(np), fwd(np * n), fwd_s(np * n), inv(np * n), inv_s(np * n), ninv(np), ninv_s(np),
      z4(np), z4_s(np), pm(np), pm_s(np), pinv(np), pinv_s(np), mneg(np), r64(np), r64_s(np), r60(np), r60_s(np);
  std::vector<int> w(np);
  for (size_t i = 0; i < np; ++i) {
    const u64 q = P[i];
    const Barrett64 b = barrett_make(q);
    p[i] = q;
    mu[i] = b.mu;
    w[i] = b.w;
    const u64 psi = primitive_root_2n(q, kLogN), ipsi = hinv(psi, q);
    u64 a = 1, bb = 1;
    for (size_t k = 0; k < n; ++k) {
      const size_t r = hbrv(k, kLogN);
      fwd[i * n + r] = a;
      inv[i * n + r] = bb;
      a = hmul(a, psi, q);
      bb = hmul(bb, ipsi, q);
    }
    for (size_t k = 0; k < n; ++k) {
      fwd_s[i * n + k] = shoup_companion(fwd[i * n + k], q);
      inv_s[i * n + k] = shoup_companion(inv[i * n + k], q);
    }
    ninv[i] = hinv(n % q, q);
    ninv_s[i] = shoup_companion(ninv[i], q);
    z4[i] = hpow(psi, n / 2, q);
    z4_s[i] = shoup_companion(z4[i], q);
    u64 pp = 1;
    for (int k = 0; k < K; ++k) pp = hmul(pp, P[L + k] % q, q);
    pm[i] = i < (size_t)L ? pp : 0;
    pm_s[i] = shoup_companion(pm[i], q);
    pinv[i] = i < (size_t)L ? hinv(pp, q) : 0;
    pinv_s[i] = shoup_companion(pinv[i], q);
    u64 qi = q;  // Newton's iteration for q^-1 mod 2^64: each step doubles the correct low bits
    for (int it = 0; it < 6; ++it) qi *= 2 - q * qi;
    mneg[i] = 0 - qi;
    r64[i] = (u64)(((u128)1 << 64) % q);
    r64_s[i] = shoup_companion(r64[i], q);
    r60[i] = (1ULL << 60) % q;
    r60_s[i] = shoup_companion(r60[i], q);
  }
  std::vector<WideConv> modup((size_t)(L + 1) * bmax), moddown((size_t)(L + 1)), rescale((size_t)(L + 1)),
      mdrs((size_t)(L + 1));
  std::vector<u64> ql((size_t)(L + 1) * L, 0), ql_s((size_t)(L + 1) * L, 0);
  for (int ell = 1; ell <= L; ++ell) {
    const int beta = (ell + alpha - 1) / alpha;
    for (int j = 0; j < beta; ++j) {
      const int lo = j * alpha, hi = std::min(lo + alpha, ell);
      std::vector<int> src, dst, slot;
      for (int i = lo; i < hi; ++i) src.push_back(i);
      for (int e = 0; e < ell + K; ++e) {
        if (e >= lo && e < hi) continue;
        dst.push_back(e < ell ? e : L + (e - ell));
        slot.push_back(e);
      }
      fill_wide_conv(modup[(size_t)ell * bmax + j], P, src, dst, slot);
    }
    std::vector<int> src, dst, slot;
    for (int k = 0; k < K; ++k) src.push_back(L + k);
    for (int i = 0; i < ell; ++i) {
      dst.push_back(i);
      slot.push_back(i);
    }
    fill_wide_conv(moddown[ell], P, src, dst, slot);
    if (ell >= 2) {  // the centered lift of q_{ell-1}: a one-source conversion (hinv = 1, factors 1)
      std::vector<int> rs_src = {ell - 1}, rs_dst, rs_slot;
      for (int i = 0; i + 1 < ell; ++i) {
        rs_dst.push_back(i);
        rs_slot.push_back(i);
      }
      fill_wide_conv(rescale[ell], P, rs_src, rs_dst, rs_slot);
      // ModDown fused with the rescale: the ModDown sums of q_0 .. q_{ell-2} times P^-1, q_{ell-1} as
      // the extra target nt (its factors times P^-1 as well), P^-1 folded into Z's inverse transform
      WideConv& fc = mdrs[ell];
      fill_wide_conv(fc, P, src, rs_dst, rs_slot);
      for (int t = 0; t <= fc.nt; ++t) {
        const int qi = t < fc.nt ? rs_dst[t] : ell - 1;
        const u64 q = P[qi];
        for (int sidx = 0; sidx < fc.ns; ++sidx) {
          u64 v = pinv[qi];
          for (int r = 0; r < fc.ns; ++r)
            if (r != sidx) v = hmul(v, P[src[r]] % q, q);
          fc.hmod[sidx][t] = v;
          fc.hmod_s[sidx][t] = shoup_companion(v, q);
          fc.hmod_m[sidx][t] = (u64)(((u128)v << 64) % q);
        }
      }
      fc.dst_prime[fc.nt] = ell - 1;
      fc.dst_slot[fc.nt] = ell - 1;
      const u64 ql = P[ell - 1], z0 = hmul(ninv[ell - 1], pinv[ell - 1], ql);
      const u64 z1 = hmul(z0, inv[(size_t)(ell - 1) * n + 1], ql);
      fc.z_n0 = z0;
      fc.z_n0_s = shoup_companion(z0, ql);
      fc.z_n1 = z1;
      fc.z_n1_s = shoup_companion(z1, ql);
    }
    for (int i = 0; i + 1 < ell; ++i) {
      const u64 v = hinv(P[ell - 1] % P[i], P[i]);
      ql[(size_t)ell * L + i] = v;
      ql_s[(size_t)ell * L + i] = shoup_companion(v, P[i]);
    }
  }

  // the fused key switch's source constants: hinv with the inverse transform's last stage folded in
  auto fold_inverse = [&](WideConv& cc) {
    for (int s = 0; s < cc.ns; ++s) {
      const int sp = cc.src_prime[s];
      const u64 b = P[sp];
      const u64 n0 = hmul(ninv[sp], cc.hinv[s], b), n1 = hmul(n0, inv[(size_t)sp * n + 1], b);
      cc.inv_n0[s] = n0;
      cc.inv_n0_s[s] = shoup_companion(n0, b);
      cc.inv_n1[s] = n1;
      cc.inv_n1_s[s] = shoup_companion(n1, b);
    }
  };
  for (WideConv& cc : modup) fold_inverse(cc);
  for (WideConv& cc : moddown) fold_inverse(cc);
  for (WideConv& cc : rescale) fold_inverse(cc);
  for (WideConv& cc : mdrs) fold_inverse(cc);

  // The matrix-core conversion's fold needs every target prime above 2^46 (|byte-position sum| < 2^45).
  bool mconv = true;
  for (size_t i = 0; i < np; ++i) mconv = mconv && P[i] > (1ULL << 46);
  std::vector<int8_t> dig;
  if (mconv) {
    for (int ell = 1; ell <= L; ++ell) {
      const int beta = (ell + alpha - 1) / alpha;
      for (int j = 0; j < beta; ++j) fill_wide_digits(modup[(size_t)ell * bmax + j], P, dig);
      fill_wide_digits(moddown[ell], P, dig);
      if (ell >= 2) fill_wide_digits(rescale[ell], P, dig);
      if (ell >= 2) fill_wide_digits(mdrs[ell], P, dig);
    }
  }

  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  struct Part {
    const void* src;
    size_t bytes;
    size_t off;
  };
  std::vector<Part> parts = {
      {p.data(), np * 8}, {mu.data(), np * 8}, {w.data(), np * sizeof(int)},
      {fwd.data(), fwd.size() * 8}, {fwd_s.data(), fwd_s.size() * 8}, {inv.data(), inv.size() * 8},
      {inv_s.data(), inv_s.size() * 8}, {ninv.data(), np * 8}, {ninv_s.data(), np * 8},
      {z4.data(), np * 8}, {z4_s.data(), np * 8}, {pm.data(), np * 8}, {pm_s.data(), np * 8},
      {pinv.data(), np * 8}, {pinv_s.data(), np * 8},
      {modup.data(), modup.size() * sizeof(WideConv)}, {moddown.data(), moddown.size() * sizeof(WideConv)},
      {ql.data(), ql.size() * 8}, {ql_s.data(), ql_s.size() * 8}, {dig.data(), dig.size()},
      {mneg.data(), np * 8}, {r64.data(), np * 8}, {r64_s.data(), np * 8},
      {rescale.data(), rescale.size() * sizeof(WideConv)}, {mdrs.data(), mdrs.size() * sizeof(WideConv)},
      {r60.data(), np * 8}, {r60_s.data(), np * 8},
  };
  size_t off = 0;
  for (Part& pt : parts) {
    pt.off = off;
    off = align(off + pt.bytes);
  }
  WideState* ws = new (std::nothrow) WideState();
  if (!ws) return HCK_ERR_ALLOC;
  hipError_t e = hipMalloc(&ws->block, off);
  if (e != hipSuccess) {
    delete ws;
    return (int)e;
  }
  char* base = (char*)ws->block;
  for (const Part& pt : parts) {
    if (pt.bytes == 0) continue;
    e = hipMemcpy(base + pt.off, pt.src, pt.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(ws->block);
      delete ws;
      return (int)e;
    }
  }
  auto at = [&](int i) { return base + parts[i].off; };
  WideTables& T = ws->t;
  T.p = (const u64*)at(0);
  T.mu = (const u64*)at(1);
  T.w = (const int*)at(2);
  T.fwd = (const u64*)at(3);
  T.fwd_s = (const u64*)at(4);
  T.inv = (const u64*)at(5);
  T.inv_s = (const u64*)at(6);
  T.ninv = (const u64*)at(7);
  T.ninv_s = (const u64*)at(8);
  T.zeta4 = (const u64*)at(9);
  T.zeta4_s = (const u64*)at(10);
  T.pmod = (const u64*)at(11);
  T.pmod_s = (const u64*)at(12);
  T.pinv = (const u64*)at(13);
  T.pinv_s = (const u64*)at(14);
  ws->modup = (WideConv*)at(15);
  ws->moddown = (WideConv*)at(16);
  ws->qlast_inv = (u64*)at(17);
  ws->qlast_inv_s = (u64*)at(18);
  ws->conv_dig = mconv ? (const void*)at(19) : nullptr;
  T.mneg = (const u64*)at(20);
  T.r64 = (const u64*)at(21);
  T.r64_s = (const u64*)at(22);
  ws->rescale = (WideConv*)at(23);
  ws->mdrs = (WideConv*)at(24);
  T.r60 = (const u64*)at(25);
  T.r60_s = (const u64*)at(26);
  ws->primes_below_2_60 = true;
  for (int i = 0; i < c->np; ++i) ws->primes_below_2_60 = ws->primes_below_2_60 && c->primes[i] < (1ULL << 60);
  c->wide = ws;
  return HCK_OK;
}

void wide_free(hck_context* c) {
  if (!c->wide) return;
  if (c->wide->block) (void)hipFree(c->wide->block);
  delete c->wide;
  c->wide = nullptr;
}

int wide_twiddles(const hck_context* c, int prime_idx, int inverse, uint64_t* out) {
  const u64* src = (inverse ? c->wide->t.inv : c->wide->t.fwd) + (size_t)prime_idx * kN;
  hipError_t e = hipMemcpy(out, src, (size_t)kN * 8, hipMemcpyDeviceToHost);
  return e == hipSuccess ? HCK_OK : (int)e;
}

// ================================================================================== entry bodies
int wide_ntt(const hck_context* c, const uint64_t* src, uint64_t* dst, int groups, long long src_stride,
             long long dst_stride, const LimbList& list, bool inverse, hipStream_t s) {
  if (list.n <= 0 || groups <= 0) return HCK_OK;
  if (list.n > kMaxList || groups > 65535) return HCK_ERR_ARG;
  const dim3 grid(16, list.n, groups);
  const WideTables& T = c->wide->t;
  if (!inverse) {
    wk_fwd_cols<<<grid, kWT, 0, s>>>(src, dst, src_stride, dst_stride, list, T);
    wk_fwd_rows<<<grid, kWT, 0, s>>>(dst, dst_stride, list, T);
  } else {
    wk_inv_rows<<<grid, kWT, 0, s>>>(src, dst, src_stride, dst_stride, list, T);
    wk_inv_cols<<<grid, kWT, 0, s>>>(dst, dst_stride, list, T);
  }
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_encode_ntt(const hck_context* c, const double* vre, const double* vim, double scale, uint64_t* out,
                    long long out_stride, int rows, int* overflow, const LimbList& list, hipStream_t s) {
  if (list.n <= 0 || rows <= 0) return HCK_OK;
  if (list.n > kMaxList || rows > 65535) return HCK_ERR_ARG;
  const int lpb = encode_limbs_per_block(list.n, rows);
  wk_encode_cols<<<dim3(16, (list.n + lpb - 1) / lpb, rows), kWT, 0, s>>>(vre, vim, scale, out, out_stride, list, lpb,
                                                                         overflow, c->wide->t);
  wk_fwd_rows<<<dim3(16, list.n, rows), kWT, 0, s>>>(out, out_stride, list, c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

namespace {
LimbList q_list(int ell, int first = 0) {
  LimbList l;
  l.n = ell - first;
  for (int i = first; i < ell; ++i) {
    l.off[i - first] = (uint16_t)i;
    l.prime[i - first] = (uint8_t)i;
  }
  return l;
}
}  // namespace

namespace {
// The base conversion of nb items: on the matrix cores (the context's default engine) when the
// context has its digit tables, else on the VALU (wk_conv); identical residues.
void launch_wconv(const hck_context* c, const u64* src, long long src_item, int src_off, u64* dst,
                  long long dst_item, const WideConv* cc, int nb, hipStream_t s) {
  const WideState& W = *c->wide;
  if (c->conv_engine == 1 && W.conv_dig) {
    if (nb >= 4)
      wk_mconv<4><<<dim3(kN / 256, nb), 256, 0, s>>>(src, src_item, src_off, dst, dst_item, cc,
                                                      (const wv4i*)W.conv_dig, W.t);
    else
      wk_mconv<1><<<dim3(kN / 64, nb), 256, 0, s>>>(src, src_item, src_off, dst, dst_item, cc,
                                                     (const wv4i*)W.conv_dig, W.t);
  } else {
    wk_conv<<<dim3(kN / 256, nb), 256, 0, s>>>(src, src_item, src_off, dst, dst_item, cc, W.t);
  }
}
}  // namespace

// Per item: X (ell) + EXT (ell + K) + ACC (2 (ell + K)) + CV (ell) + SD (ell) + S0 (ell) limbs.
size_t wide_ks_bytes(const hck_context* c, int ell, int batch) {
  if (wide_fused_ok(c)) return wide_fused_bytes(c, ell, batch);
  // per item: X [ell], EXT [beta][ell + K], ACC [2][ell + K], CV, SD, S0 [ell] each
  const size_t nb = (size_t)std::min(batch, kWideChunk), ext_l = (size_t)(ell + c->K);
  return nb * (size_t)kN * 8 * (4 * (size_t)ell + ((size_t)beta_of(c, ell) + 2) * ext_l);
}

int wide_ks(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
            const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
            const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
            char* ws, hipStream_t s, uint64_t* ext_b, uint64_t* ext_a, long long ext_stride,
            const uint32_t* galois_items) {
  if (wide_fused_ok(c))
    return wide_ks_fused(c, ell, batch, d, d_stride, galois, ksk, add, add_stride, acc_b, acc_a, acc_stride, out_b,
                         out_a, out_stride, ws, s, ext_b, ext_a, ext_stride, galois_items);
  if (c->alpha > kMaxAlpha || ell + c->K > kMaxList) return HCK_ERR_UNSUPPORTED;
  const WideState& W = *c->wide;
  const WideTables& T = W.t;
  const int K = c->K, L = c->L, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN;
  const bool permute = galois_items != nullptr || galois != 1u;
  const LimbList lq = q_list(ell);
  LimbList lp;
  lp.n = K;
  for (int k = 0; k < K; ++k) {
    lp.off[k] = (uint16_t)(ell + k);
    lp.prime[k] = (uint8_t)(L + k);
  }
  for (int b0 = 0; b0 < batch; b0 += kWideChunk) {
    const int nb = std::min(kWideChunk, batch - b0);
    u64* X = (u64*)ws;
    u64* EXT = X + (long long)nb * ell * n;                  // [nb][beta][ext_l]
    const long long ext_item = (long long)beta * ext_l * n;
    u64* ACC = EXT + (long long)nb * ext_item;
    u64* CV = ACC + (long long)nb * 2 * ext_l * n;
    u64* SD = CV + (long long)nb * ell * n;
    u64* S0 = SD + (long long)nb * ell * n;
    const u64* dd = d + (long long)b0 * d_stride;
    long long dd_item = d_stride;
    const u64* a0 = add ? add + (long long)b0 * add_stride : nullptr;
    long long a0_item = add_stride;
    if (permute) {
      WGal G{};
      for (int b = 0; b < nb; ++b) G.g[b] = galois_items ? galois_items[b0 + b] : galois;
      wk_automorph<<<dim3(kN / 256, ell, nb), 256, 0, s>>>(dd, dd_item, SD, (long long)ell * n, G);
      dd = SD;
      dd_item = (long long)ell * n;
      if (a0) {
        wk_automorph<<<dim3(kN / 256, ell, nb), 256, 0, s>>>(a0, a0_item, S0, (long long)ell * n, G);
        a0 = S0;
        a0_item = (long long)ell * n;
      }
      HCK_CHECK_LAUNCH();
    }
    int rc = wide_ntt(c, dd, X, nb, dd_item, (long long)ell * n, lq, true, s);
    if (rc) return rc;
    WKeys kp{};
    for (int b = 0; b < nb; ++b) kp.k[b] = ksk[b0 + b];
    // every digit's ModUp into its own slab, then one inner product over all of them: the
    // accumulators are written once instead of read and written per digit
    for (int j = 0; j < beta; ++j) {
      const int lo = j * alpha, hi = std::min(lo + alpha, ell);
      u64* EXTj = EXT + (long long)j * ext_l * n;
      launch_wconv(c, X, (long long)ell * n, lo, EXTj, ext_item, W.modup + (size_t)ell * bmax + j, nb, s);
      HCK_CHECK_LAUNCH();
      LimbList le;
      le.n = 0;
      for (int e = 0; e < ext_l; ++e) {
        if (e >= lo && e < hi) continue;
        le.off[le.n] = (uint16_t)e;
        le.prime[le.n] = (uint8_t)(e < ell ? e : L + (e - ell));
        ++le.n;
      }
      // the column pass only: the inner product finishes each digit's transform on chip
      wk_fwd_cols<<<dim3(16, le.n, nb), kWT, 0, s>>>(EXTj, EXTj, ext_item, ext_item, le, T);
      HCK_CHECK_LAUNCH();
    }
    wk_ks_ip_rows<<<dim3(16, ext_l, nb), kWT, 0, s>>>(EXT, ext_item, dd, dd_item, alpha, beta, kp, ell, L, K, bmax,
                                                      ACC, 2LL * ext_l * n, T);
    HCK_CHECK_LAUNCH();
    if (ext_b) {
      const long long ai = (long long)b0 * acc_stride, ei = (long long)b0 * ext_stride;
      wk_ks_ext_out<<<dim3(kN / 256, ext_l, nb), 256, 0, s>>>(ACC, 2LL * ext_l * n, a0, a0_item,
                                                              acc_b ? acc_b + ai : nullptr, acc_stride, ext_b + ei,
                                                              ext_stride, ell, L, T);
      wk_ks_ext_out<<<dim3(kN / 256, ext_l, nb), 256, 0, s>>>(ACC + (long long)ext_l * n, 2LL * ext_l * n, nullptr, 0,
                                                              acc_a ? acc_a + ai : nullptr, acc_stride, ext_a + ei,
                                                              ext_stride, ell, L, T);
      HCK_CHECK_LAUNCH();
      continue;
    }
    for (int comp = 0; comp < 2; ++comp) {
      u64* A = ACC + (long long)comp * ext_l * n;
      rc = wide_ntt(c, A, A, nb, 2LL * ext_l * n, 2LL * ext_l * n, lp, true, s);
      if (rc) return rc;
      launch_wconv(c, A, 2LL * ext_l * n, ell, CV, (long long)ell * n, W.moddown + ell, nb, s);
      HCK_CHECK_LAUNCH();
      rc = wide_ntt(c, CV, CV, nb, (long long)ell * n, (long long)ell * n, lq, false, s);
      if (rc) return rc;
      const u64* accin = comp == 0 ? acc_b : acc_a;
      u64* o = (comp == 0 ? out_b : out_a) + (long long)b0 * out_stride;
      wk_ks_out<<<dim3(kN / 256, ell, nb), 256, 0, s>>>(
          A, 2LL * ext_l * n, CV, (long long)ell * n, comp == 0 ? a0 : nullptr, a0_item,
          accin ? accin + (long long)b0 * acc_stride : nullptr, acc_stride, o, out_stride, T.pinv, T.pinv_s, T);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

size_t wide_hoist_bytes(const hck_context* c, int ell, int inputs) {
  if (wide_fused_ok(c)) return wide_fused_hoist_bytes(c, ell, inputs);
  return (size_t)std::min(inputs, kWideChunk) * kN * 8 * (size_t)ell;
}

int wide_hoist(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride, uint64_t* digits,
               char* ws, hipStream_t s) {
  if (wide_fused_ok(c)) return wide_hoist_fused(c, ell, inputs, d, d_stride, digits, ws, s);
  if (c->alpha > kMaxAlpha || ell + c->K > kMaxList) return HCK_ERR_UNSUPPORTED;
  const WideState& W = *c->wide;
  const WideTables& T = W.t;
  const int K = c->K, L = c->L, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN, dig_item = (long long)beta * ext_l * n;
  const LimbList lq = q_list(ell);
  for (int b0 = 0; b0 < inputs; b0 += kWideChunk) {
    const int nb = std::min(kWideChunk, inputs - b0);
    u64* X = (u64*)ws;
    const u64* dd = d + (long long)b0 * d_stride;
    int rc = wide_ntt(c, dd, X, nb, d_stride, (long long)ell * n, lq, true, s);
    if (rc) return rc;
    for (int j = 0; j < beta; ++j) {
      const int lo = j * alpha, hi = std::min(lo + alpha, ell);
      u64* EXT = digits + (long long)b0 * dig_item + (long long)j * ext_l * n;
      launch_wconv(c, X, (long long)ell * n, lo, EXT, dig_item, W.modup + (size_t)ell * bmax + j, nb, s);
      HCK_CHECK_LAUNCH();
      LimbList le;
      le.n = 0;
      for (int e = 0; e < ext_l; ++e) {
        if (e >= lo && e < hi) continue;
        le.off[le.n] = (uint16_t)e;
        le.prime[le.n] = (uint8_t)(e < ell ? e : L + (e - ell));
        ++le.n;
      }
      rc = wide_ntt(c, EXT, EXT, nb, dig_item, dig_item, le, false, s);
      if (rc) return rc;
      // the digit's own limbs are the input's NTT-domain limbs themselves
      hipError_t e = hipMemcpy2DAsync(EXT + (long long)lo * n, (size_t)dig_item * 8, dd + (long long)lo * n,
                                      (size_t)d_stride * 8, (size_t)(hi - lo) * n * 8, (size_t)nb,
                                      hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return (int)e;
    }
  }
  return HCK_OK;
}

size_t wide_hoisted_bytes(const hck_context* c, int ell, int items) {
  if (wide_fused_ok(c)) return wide_fused_hoisted_bytes(c, ell, items);
  // ACC [2][ell + K] + CV [ell] + sigma(c0) [ell] per item of a launch
  return (size_t)std::min(items, kWideChunk) * kN * 8 * (size_t)(2 * (ell + c->K) + 2 * ell);
}

int wide_hoisted(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
                 const uint64_t* const* ksk, const uint64_t* c0, const uint64_t* c1, long long in_stride,
                 const uint64_t* digits, uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws,
                 hipStream_t s) {
  if (wide_fused_ok(c))
    return wide_hoisted_fused(c, ell, inputs, items, galois, ksk, c0, in_stride, digits, out_b, out_a, out_stride, ws, s);
  (void)c1;  // its ModUp is in `digits`
  if (c->alpha > kMaxAlpha || ell + c->K > kMaxList) return HCK_ERR_UNSUPPORTED;
  const WideState& W = *c->wide;
  const WideTables& T = W.t;
  const int K = c->K, L = c->L, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN;
  const LimbList lq = q_list(ell);
  LimbList lp;
  lp.n = K;
  for (int k = 0; k < K; ++k) {
    lp.off[k] = (uint16_t)(ell + k);
    lp.prime[k] = (uint8_t)(L + k);
  }
  for (int i0 = 0; i0 < items; i0 += kWideChunk) {
    const int nb = std::min(kWideChunk, items - i0);
    u64* ACC = (u64*)ws;
    u64* CV = ACC + (long long)nb * 2 * ext_l * n;
    u64* S0 = CV + (long long)nb * ell * n;
    WGal G{};
    WKeys kp{};
    for (int b = 0; b < nb; ++b) {
      G.g[b] = galois[i0 + b];
      kp.k[b] = ksk[i0 + b];
    }
    const int first = i0 % inputs;
    wk_ks_ip_h<<<dim3(kN / 256, ext_l, nb), 256, 0, s>>>(digits, inputs, first, G, kp, beta, ell, L, K, bmax, ACC,
                                                         2LL * ext_l * n, T);
    wk_automorph_h<<<dim3(kN / 256, ell, nb), 256, 0, s>>>(c0, in_stride, inputs, first, S0, (long long)ell * n, G);
    HCK_CHECK_LAUNCH();
    for (int comp = 0; comp < 2; ++comp) {
      u64* A = ACC + (long long)comp * ext_l * n;
      int rc = wide_ntt(c, A, A, nb, 2LL * ext_l * n, 2LL * ext_l * n, lp, true, s);
      if (rc) return rc;
      launch_wconv(c, A, 2LL * ext_l * n, ell, CV, (long long)ell * n, W.moddown + ell, nb, s);
      HCK_CHECK_LAUNCH();
      rc = wide_ntt(c, CV, CV, nb, (long long)ell * n, (long long)ell * n, lq, false, s);
      if (rc) return rc;
      u64* o = (comp == 0 ? out_b : out_a) + (long long)i0 * out_stride;
      wk_ks_out<<<dim3(kN / 256, ell, nb), 256, 0, s>>>(A, 2LL * ext_l * n, CV, (long long)ell * n,
                                                        comp == 0 ? S0 : nullptr, (long long)ell * n, nullptr, 0, o,
                                                        out_stride, T.pinv, T.pinv_s, T);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

size_t wide_moddown_bytes(const hck_context* c, int ell, int polys) {
  if (wide_fused_ok(c)) return wide_fused_moddown_bytes(c, ell, polys);
  return (size_t)polys * kN * 8 * (size_t)(c->K + ell);
}

int wide_moddown(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                 long long out_stride, char* ws, hipStream_t s) {
  if (wide_fused_ok(c)) return wide_moddown_fused(c, ell, polys, in, in_stride, out, out_stride, ws, s);
  const WideState& W = *c->wide;
  const int K = c->K, L = c->L;
  const long long n = kN;
  u64* TP = (u64*)ws;
  u64* CV = TP + (long long)polys * K * n;
  LimbList lp;
  lp.n = K;
  for (int k = 0; k < K; ++k) {
    lp.off[k] = (uint16_t)k;
    lp.prime[k] = (uint8_t)(L + k);
  }
  int rc = wide_ntt(c, in + (long long)ell * n, TP, polys, in_stride, (long long)K * n, lp, true, s);
  if (rc) return rc;
  launch_wconv(c, TP, (long long)K * n, 0, CV, (long long)ell * n, W.moddown + ell, polys, s);
  HCK_CHECK_LAUNCH();
  rc = wide_ntt(c, CV, CV, polys, (long long)ell * n, (long long)ell * n, q_list(ell), false, s);
  if (rc) return rc;
  wk_ks_out<<<dim3(kN / 256, ell, polys), 256, 0, s>>>(in, in_stride, CV, (long long)ell * n, nullptr, 0, nullptr, 0,
                                                       out, out_stride, W.t.pinv, W.t.pinv_s, W.t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t wide_rescale_bytes(const hck_context* c, int ell, int polys) {
  if (wide_fused_ok(c)) return wide_fused_rescale_bytes(c, ell, polys);
  return (size_t)polys * kN * 8 * (size_t)ell;
}

int wide_rescale(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                 long long out_stride, char* ws, hipStream_t s) {
  if (wide_fused_ok(c) && ell >= 2) return wide_rescale_fused(c, ell, polys, in, in_stride, out, out_stride, ws, s);
  const WideState& W = *c->wide;
  const long long n = kN;
  const int nt = ell - 1;
  u64* TL = (u64*)ws;
  u64* TT = TL + (long long)polys * n;
  LimbList l1;
  l1.n = 1;
  l1.off[0] = 0;
  l1.prime[0] = (uint8_t)(ell - 1);
  int rc = wide_ntt(c, in + (long long)(ell - 1) * n, TL, polys, in_stride, n, l1, true, s);
  if (rc) return rc;
  wk_lift<<<dim3(kN / 256, nt, polys), 256, 0, s>>>(TL, n, ell - 1, TT, (long long)nt * n, 0, W.t);
  HCK_CHECK_LAUNCH();
  rc = wide_ntt(c, TT, TT, polys, (long long)nt * n, (long long)nt * n, q_list(nt), false, s);
  if (rc) return rc;
  const size_t lv = (size_t)ell * c->L;
  wk_ks_out<<<dim3(kN / 256, nt, polys), 256, 0, s>>>(in, in_stride, TT, (long long)nt * n, nullptr, 0, nullptr, 0, out,
                                                      out_stride, W.qlast_inv + lv, W.qlast_inv_s + lv, W.t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t wide_modraise_bytes(const hck_context* c, int to, int polys) {
  (void)c;
  (void)to;
  return (size_t)polys * kN * 8;
}

int wide_modraise(const hck_context* c, int to, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                  long long out_stride, char* ws, hipStream_t s) {
  const long long n = kN;
  u64* TL = (u64*)ws;
  LimbList l0;
  l0.n = 1;
  l0.off[0] = 0;
  l0.prime[0] = 0;
  int rc = wide_ntt(c, in, TL, polys, in_stride, n, l0, true, s);
  if (rc) return rc;
  // a single poly may come with any item stride (0 included): its pitch is then the row itself
  const long long os = polys > 1 ? out_stride : (long long)to * n;
  wk_lift<<<dim3(kN / 256, to - 1, polys), 256, 0, s>>>(TL, n, 0, out, os, 1, c->wide->t);
  HCK_CHECK_LAUNCH();
  rc = wide_ntt(c, out, out, polys, os, os, q_list(to, 1), false, s);
  if (rc) return rc;
  const size_t row = (size_t)n * 8;
  const size_t dp = polys > 1 ? (size_t)out_stride * 8 : row, sp = polys > 1 ? (size_t)in_stride * 8 : row;
  hipError_t e = hipMemcpy2DAsync(out, dp, in, sp, row, polys, hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? HCK_OK : (int)e;
}

int wide_poly_op(const hck_context* c, int op, uint64_t* out, const uint64_t* a, const uint64_t* b, int polys,
                 long long out_stride, long long a_stride, long long b_stride, int limbs, const int* prime_idx,
                 const uint64_t* scalar, hipStream_t s) {
  WPrimeMap pm{};
  WScalars sc{};
  const bool with_scalar = op == HCK_OP_MUL_SCALAR || op == HCK_OP_ADD_SCALAR;
  for (int i = 0; i < limbs; ++i) {
    pm.prime[i] = (uint8_t)prime_idx[i];
    if (with_scalar) {
      const u64 q = c->primes[prime_idx[i]];
      sc.s[i] = scalar[i];
      sc.ss[i] = shoup_companion(scalar[i], q);
    }
  }
  const dim3 grid(kN / 256, limbs, polys);
  const WideTables& T = c->wide->t;
  switch (op) {
    case HCK_OP_ADD: wk_poly_op<HCK_OP_ADD><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_SUB: wk_poly_op<HCK_OP_SUB><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_MUL: wk_poly_op<HCK_OP_MUL><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_NEG: wk_poly_op<HCK_OP_NEG><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_MUL_SCALAR: wk_poly_op<HCK_OP_MUL_SCALAR><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_MUL_XHALF: wk_poly_op<HCK_OP_MUL_XHALF><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_MAC: wk_poly_op<HCK_OP_MAC><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    case HCK_OP_ADD_SCALAR: wk_poly_op<HCK_OP_ADD_SCALAR><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sc, T); break;
    default: return HCK_ERR_ARG;
  }
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_tensor(const hck_context* c, int ell, int batch, const uint64_t* a0, const uint64_t* a1, long long a_stride,
                const uint64_t* b0, const uint64_t* b1, long long b_stride, uint64_t* d0, uint64_t* d1, uint64_t* d2,
                long long d_stride, hipStream_t s) {
  wk_tensor<<<dim3(kN / 256, ell, batch), 256, 0, s>>>(a0, a1, a_stride, b0, b1, b_stride, d0, d1, d2, d_stride, 0,
                                                       c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_tensor_d2(const hck_context* c, int ell, int batch, const uint64_t* a0, const uint64_t* a1,
                   long long a_stride, const uint64_t* b0, const uint64_t* b1, long long b_stride, uint64_t* d0,
                   uint64_t* d1, uint64_t* d2, long long d_stride, hipStream_t s) {
  wk_tensor<<<dim3(kN / 256, ell, batch), 256, 0, s>>>(a0, a1, a_stride, b0, b1, b_stride, d0, d1, d2, d_stride,
                                                       ell - 1, c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_weighted_sum(const hck_context* c, int limbs, int n, int groups, const uint64_t* in, long long in_stride,
                      const uint64_t* w, uint64_t* out, long long out_stride, hipStream_t s) {
  wk_weighted_sum<<<dim3(kN / 256, limbs, groups), 256, 0, s>>>(in, in_stride, n, w, out, out_stride, limbs,
                                                                c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_lincomb(const hck_context* c, int limbs, int groups, int terms, const uint64_t* const* x, const uint64_t* w,
                 uint64_t* const* out, hipStream_t s) {
  if (groups > kWLcMaxGroups || (long long)groups * terms > kWLcMaxPtrs) return HCK_ERR_ARG;
  WLcPtrs P{};
  for (int j = 0; j < groups * terms; ++j) P.x[j] = x[j];
  for (int g = 0; g < groups; ++g) P.out[g] = out[g];
  wk_lincomb<<<dim3(kN / 256, limbs, groups), 256, 0, s>>>(P, terms, w, limbs, c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int wide_bsgs_mac(const hck_context* c, int limbs, const int* prime_idx, int inputs, int babies, int giants,
                  const uint64_t* const* baby_c0, const uint64_t* const* baby_c1, long long baby_stride,
                  const uint64_t* pts, long long pt_stride, uint64_t* res, hipStream_t s) {
  if (babies > kWMaxBabies) return HCK_ERR_ARG;
  WMac P{};
  for (int b = 0; b < babies; ++b) {
    if (!baby_c0[b] || !baby_c1[b]) return HCK_ERR_ARG;
    P.c0[b] = baby_c0[b];
    P.c1[b] = baby_c1[b];
  }
  WPrimeMap pm{};
  for (int l = 0; l < limbs; ++l) pm.prime[l] = (uint8_t)prime_idx[l];
  const int units_per_limb = kN / kWMacThreads;
  const int total_units = limbs * units_per_limb;
  const long long units_padded = ((long long)total_units + kXcds - 1) / kXcds * kXcds;
  bool split = true;  // the split MAC needs every prime of the launch below 2^60
  for (int l = 0; l < limbs; ++l) split = split && c->primes[prime_idx[l]] < (1ULL << 60);
  if (split) {
    const int tiles_i = (inputs + kSTI - 1) / kSTI, tiles_g = (giants + kSTG - 1) / kSTG;
    const long long blocks = units_padded * tiles_i * tiles_g;
    if (blocks > 0x7fffffffLL) return HCK_ERR_ARG;
    wk_bsgs_mac30<<<dim3((unsigned)blocks), kWMacThreads, 0, s>>>(P, baby_stride, pts, pt_stride, res, inputs, babies,
                                                                 giants, limbs, pm, units_per_limb, tiles_i, tiles_g,
                                                                 total_units, c->wide->t);
    HCK_CHECK_LAUNCH();
    return HCK_OK;
  }
  const int tiles_i = (inputs + kWTI - 1) / kWTI, tiles_g = (giants + kWTG - 1) / kWTG;
  const long long blocks = units_padded * tiles_i * tiles_g;
  if (blocks > 0x7fffffffLL) return HCK_ERR_ARG;
  wk_bsgs_mac<<<dim3((unsigned)blocks), kWMacThreads, 0, s>>>(P, baby_stride, pts, pt_stride, res, inputs, babies,
                                                             giants, limbs, pm, units_per_limb, tiles_i, tiles_g,
                                                             total_units, c->wide->t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

}  // namespace hck
