// BSGS baby-step multiply-accumulate over many inputs at once.
//
//   res[c][g][i][l][n] = sum_{b < nb} pt[g * nb + b][l][n] * baby_b[i][c][l][n]   (mod q_l)
//
// for inputs i < ni, giants g < G, components c in {0, 1}: the partial sums of the diagonal
// method that the giant steps then rotate and add (exact-residue semantics of
// bench/cmp/kernels/holmes_mac.cu:8-12, multi-input tiling of holmes_mac.cu:108-190).
//
// A thread owns one coefficient of one limb and a TI x TG tile of (input, giant) accumulators for
// both components: per baby step it reads TG plaintext words and 2 TI baby words for 2 TI TG
// products (the next step's words are loaded while the current step computes), so plaintexts
// stream once per input tile and babies once per giant tile.  All tiles
// of one (limb, 128-coefficient) unit are dispatched to the same XCD (workgroups are handed to
// the 8 XCDs round-robin by linear id), so the unit's plaintext and baby data is fetched from HBM
// once and then served from that XCD's L2.
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"
#include "modarith64.hpp"

namespace hck {
namespace {

constexpr int kMacThreads = 128;
// Register tile: inputs x giants per thread (both components).  Tunable at build time.
#ifndef HCK_MAC_TI
#define HCK_MAC_TI 4
#endif
#ifndef HCK_MAC_TG
#define HCK_MAC_TG 8
#endif
constexpr int kTI = HCK_MAC_TI;
constexpr int kTG = HCK_MAC_TG;
constexpr int kMaxBabies = 64;

struct BabyPtrs {
  const uint64_t* c0[kMaxBabies];
  const uint64_t* c1[kMaxBabies];
};
struct MacPrimes {
  uint8_t prime[kMaxPrimes];
};

// One baby step's operands for a thread: TG plaintext words, TI words of each component.
struct MacOps {
  uint64_t w[kTG], x0[kTI], x1[kTI];
};

__device__ __forceinline__ void mac_load(MacOps& o, const BabyPtrs& babies, int b, int nb, int G, int ni,
                                         int g0, int i0, const uint64_t* __restrict__ pts, long long pt_stride,
                                         long long baby_stride, long long ln) {
#pragma unroll
  for (int g = 0; g < kTG; ++g) {
    const int gg = g0 + g < G ? g0 + g : g0;  // clamp: duplicates are never stored
    o.w[g] = pts[((long long)gg * nb + b) * pt_stride + ln];
  }
  const uint64_t* b0 = babies.c0[b];
  const uint64_t* b1 = babies.c1[b];
#pragma unroll
  for (int t = 0; t < kTI; ++t) {
    const int ii = i0 + t < ni ? i0 + t : i0;
    o.x0[t] = b0[(long long)ii * baby_stride + ln];
    o.x1[t] = b1[(long long)ii * baby_stride + ln];
  }
}

__global__ __launch_bounds__(kMacThreads) void k_bsgs_mac(uint64_t* __restrict__ res, BabyPtrs babies,
                                                          long long baby_stride, int nb, int ni, int G,
                                                          const uint64_t* __restrict__ pts, long long pt_stride,
                                                          int limbs, MacPrimes mp, int units_per_limb,
                                                          int tiles_i, int tiles_g, int total_units, DevTables T) {
  // XCD-aware decode of the linear workgroup id into (unit, tile)
  const int tiles = tiles_i * tiles_g;
  const int lin = blockIdx.x;
  const int xcd = lin % kXcds, k = lin / kXcds;
  const int unit = (k / tiles) * kXcds + xcd;
  const int tile = k % tiles;
  if (unit >= total_units) return;
  const int l = unit / units_per_limb;
  const int n = (unit % units_per_limb) * kMacThreads + threadIdx.x;
  const int i0 = (tile % tiles_i) * kTI, g0 = (tile / tiles_i) * kTG;
  const int pi = mp.prime[l];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const long long ln = (long long)l * kN + n;
  double acc[kTI][2][kTG];
#pragma unroll
  for (int t = 0; t < kTI; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kTG; ++g) acc[t][c][g] = 0.0;
  // one baby step's products from its loaded words; every 8 steps the sums are reduced
  auto step = [&](const MacOps& cur, int b) {
    double w[kTG], wp[kTG];
#pragma unroll
    for (int g = 0; g < kTG; ++g) {
      w[g] = u2d(cur.w[g]);
      wp[g] = w[g] * pinv;
    }
#pragma unroll
    for (int t = 0; t < kTI; ++t) {
      const double x0 = u2d(cur.x0[t]), x1 = u2d(cur.x1[t]);
#pragma unroll
      for (int g = 0; g < kTG; ++g) {
        acc[t][0][g] += mulc(x0, w[g], wp[g], p);  // canonical operands: |term| <= 0.875 p
        acc[t][1][g] += mulc(x1, w[g], wp[g], p);
      }
    }
    if ((b & 7) == 7) {
#pragma unroll
      for (int t = 0; t < kTI; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int g = 0; g < kTG; ++g) acc[t][c][g] = reduce(acc[t][c][g], p, pinv);
    }
  };
  // two-stage software pipeline on two register sets: baby step b + 1's words load into one set while
  // step b computes from the other (the last pair reloads its own words, unused), so the wait before
  // a step's products covers only that step's own loads.
  MacOps o0, o1;
  mac_load(o0, babies, 0, nb, G, ni, g0, i0, pts, pt_stride, baby_stride, ln);
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    mac_load(o1, babies, b + 1, nb, G, ni, g0, i0, pts, pt_stride, baby_stride, ln);
    // the loads stay ahead of the products they overlap: neither the compiler's IR passes (the
    // memory clobber) nor the scheduler (the barrier) move them below
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o0, b);
    mac_load(o0, babies, b + 2 < nb ? b + 2 : b + 1, nb, G, ni, g0, i0, pts, pt_stride, baby_stride, ln);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    step(o1, b + 1);
  }
  if (b < nb) step(o0, b);  // odd count: the last step's words are in o0
  const long long is = (long long)limbs * kN, gs = (long long)ni * is, cs = (long long)G * gs;
#pragma unroll
  for (int t = 0; t < kTI; ++t) {
    if (i0 + t >= ni) break;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kTG; ++g)
        if (g0 + g < G)
          res[c * cs + (long long)(g0 + g) * gs + (long long)(i0 + t) * is + ln] = d2u(canon(acc[t][c][g], p, pinv));
  }
}

// ----------------------------------------------------------------- the sidecar-shaped MAC
// holmes_mac_multi's layout (bench/cmp/kernels/holmes_mac.cu:359-402): one device pointer per input to
// its baby basis [nb][>= limbs][N] (baby stride bstride words), plaintext rows [groups * nb][>= limbs][N]
// (row stride pstride), res [2][groups][inputs][limbs][N], and the moduli as a device array (limb l uses
// primes[l]).  No context handle is needed: every workgroup derives its limb's Barrett constant from
// the prime (modarith64.hpp), so the entry works for any prime below 2^62 -- the reference's 59/60-bit
// chains included.  Products are reduced one by one and summed canonically.
constexpr int kAbiMaxInputs = 32;
constexpr int kAbiThreads = 128;
constexpr int kAbiTI = 2;
constexpr int kAbiTG = 8;

struct AbiInputs {
  const uint64_t* c0[kAbiMaxInputs];
  const uint64_t* c1[kAbiMaxInputs];
};

__global__ __launch_bounds__(kAbiThreads) void k_mac_multi_abi(uint64_t* __restrict__ res, AbiInputs in,
                                                               long long bstride, int nb, int ni, int G,
                                                               const uint64_t* __restrict__ pts, long long pstride,
                                                               int limbs, const uint64_t* __restrict__ primes,
                                                               int tiles_i) {
  const int l = blockIdx.y;
  const int units = kN / kAbiThreads;
  const int unit = blockIdx.x % units, tile = blockIdx.x / units;
  const int i0 = (tile % tiles_i) * kAbiTI, g0 = (tile / tiles_i) * kAbiTG;
  const long long ln = (long long)l * kN + unit * kAbiThreads + threadIdx.x;
  const Barrett64 br = barrett_make(primes[l]);
  const uint64_t p = br.p;
  uint64_t acc[kAbiTI][2][kAbiTG];
#pragma unroll
  for (int t = 0; t < kAbiTI; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kAbiTG; ++g) acc[t][c][g] = 0;
  for (int b = 0; b < nb; ++b) {
    uint64_t w[kAbiTG];
#pragma unroll
    for (int g = 0; g < kAbiTG; ++g) {
      const int gg = g0 + g < G ? g0 + g : g0;  // clamped rows are computed but never stored
      w[g] = pts[((long long)gg * nb + b) * pstride + ln];
    }
#pragma unroll
    for (int t = 0; t < kAbiTI; ++t) {
      const int ii = i0 + t < ni ? i0 + t : i0;
      const uint64_t x0 = in.c0[ii][(long long)b * bstride + ln];
      const uint64_t x1 = in.c1[ii][(long long)b * bstride + ln];
#pragma unroll
      for (int g = 0; g < kAbiTG; ++g) {
        acc[t][0][g] = addmod64(acc[t][0][g], mulmod64(x0, w[g], br), p);
        acc[t][1][g] = addmod64(acc[t][1][g], mulmod64(x1, w[g], br), p);
      }
    }
  }
  const long long is = (long long)limbs * kN, gs = (long long)ni * is, cs = (long long)G * gs;
#pragma unroll
  for (int t = 0; t < kAbiTI; ++t) {
    if (i0 + t >= ni) break;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kAbiTG; ++g)
        if (g0 + g < G) res[c * cs + (long long)(g0 + g) * gs + (long long)(i0 + t) * is + ln] = acc[t][c][g];
  }
}

}  // namespace
}  // namespace hck

extern "C" int holmes_mac_multi(uint64_t* res, const uint64_t* const* c0s, const uint64_t* const* c1s,
                                long long bstride, int nb, int inputs, const uint64_t* pts, long long pstride,
                                int groups, int ti, int limbs, const uint64_t* primes, const uint64_t* ratios,
                                const uint64_t* ks, void* stream) {
  (void)ratios;  // the caller's Barrett tables: this entry derives its constants from `primes`
  (void)ks;
  if (inputs < 1 || inputs > hck::kAbiMaxInputs) return -1;
  if (nb < 1) return -2;
  if (groups < 1 || groups > 16 || (groups > 8 && ti != 10116)) return -3;
  static const int kTiles[] = {1, 2, 4, 404, 408, 802, 804, 1601, 1602, 10108, 10116, 10204, 10208, 10402, 10404};
  bool known = false;
  for (int v : kTiles) known |= v == ti;
  if (!known) return -4;  // the reference's tile selector is validated, the tile here is this kernel's own
  if (!res || !c0s || !c1s || !pts || !primes || limbs < 1 || limbs > 65535) return HCK_ERR_ARG;
  hck::AbiInputs in{};
  for (int i = 0; i < inputs; ++i) {
    if (!c0s[i] || !c1s[i]) return HCK_ERR_ARG;
    in.c0[i] = c0s[i];
    in.c1[i] = c1s[i];
  }
  const int tiles_i = (inputs + hck::kAbiTI - 1) / hck::kAbiTI;
  const int tiles_g = (groups + hck::kAbiTG - 1) / hck::kAbiTG;
  const dim3 grid((unsigned)(hck::kN / hck::kAbiThreads * tiles_i * tiles_g), (unsigned)limbs);
  hck::k_mac_multi_abi<<<grid, hck::kAbiThreads, 0, (hipStream_t)stream>>>(res, in, bstride, nb, inputs, groups,
                                                                           pts, pstride, limbs, primes, tiles_i);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

extern "C" int hck_bsgs_mac(const hck_context* ctx, int limbs, const int* prime_idx, int inputs, int babies,
                            int giants, const uint64_t* const* baby_c0, const uint64_t* const* baby_c1,
                            int64_t baby_stride, const uint64_t* pts, int64_t pt_stride, uint64_t* res,
                            void* stream) {
  if (!ctx || !prime_idx || !baby_c0 || !baby_c1 || !pts || !res) return HCK_ERR_ARG;
  if (limbs < 1 || limbs > hck::kMaxPrimes || inputs < 1 || babies < 1 || babies > hck::kMaxBabies || giants < 1)
    return HCK_ERR_ARG;
  hck::MacPrimes mp{};
  for (int l = 0; l < limbs; ++l) {
    if (prime_idx[l] < 0 || prime_idx[l] >= ctx->np) return HCK_ERR_ARG;
    mp.prime[l] = (uint8_t)prime_idx[l];
  }
  if (ctx->wide)
    return hck::wide_bsgs_mac(ctx, limbs, prime_idx, inputs, babies, giants, baby_c0, baby_c1, baby_stride, pts,
                              pt_stride, res, (hipStream_t)stream);
  hck::BabyPtrs bp{};
  for (int b = 0; b < babies; ++b) {
    if (!baby_c0[b] || !baby_c1[b]) return HCK_ERR_ARG;
    bp.c0[b] = baby_c0[b];
    bp.c1[b] = baby_c1[b];
  }
  const int units_per_limb = hck::kN / hck::kMacThreads;
  const int total_units = limbs * units_per_limb;
  const int tiles_i = (inputs + hck::kTI - 1) / hck::kTI, tiles_g = (giants + hck::kTG - 1) / hck::kTG;
  const int tiles = tiles_i * tiles_g;
  const long long units_padded = ((long long)total_units + hck::kXcds - 1) / hck::kXcds * hck::kXcds;
  const long long blocks = units_padded * tiles;
  if (blocks > 0x7fffffffLL) return HCK_ERR_ARG;
  hck::k_bsgs_mac<<<dim3((unsigned)blocks), hck::kMacThreads, 0, (hipStream_t)stream>>>(
      res, bp, baby_stride, babies, inputs, giants, pts, pt_stride, limbs, mp, units_per_limb, tiles_i, tiles_g,
      total_units, ctx->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}
