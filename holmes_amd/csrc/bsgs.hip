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
// products, so plaintexts stream once per input tile and babies once per giant tile.  All tiles
// of one (limb, 128-coefficient) unit are dispatched to the same XCD (workgroups are handed to
// the 8 XCDs round-robin by linear id), so the unit's plaintext and baby data is fetched from HBM
// once and then served from that XCD's L2.
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"

namespace hck {
namespace {

constexpr int kMacThreads = 128;
constexpr int kTI = 4;          // inputs per thread
constexpr int kTG = 4;          // giants per thread
constexpr int kMaxBabies = 64;

struct BabyPtrs {
  const uint64_t* c0[kMaxBabies];
  const uint64_t* c1[kMaxBabies];
};

__global__ __launch_bounds__(kMacThreads) void k_bsgs_mac(uint64_t* __restrict__ res, BabyPtrs babies,
                                                          long long baby_stride, int nb, int ni, int G,
                                                          const uint64_t* __restrict__ pts, long long pt_stride,
                                                          int limbs, int units_per_limb, int tiles_i, int tiles_g,
                                                          int total_units, DevTables T) {
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
  const double p = T.p[l], pinv = T.pinv[l];
  const long long ln = (long long)l * kN + n;
  double acc[kTI][2][kTG];
#pragma unroll
  for (int t = 0; t < kTI; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < kTG; ++g) acc[t][c][g] = 0.0;
  for (int b = 0; b < nb; ++b) {
    double w[kTG], wp[kTG];
#pragma unroll
    for (int g = 0; g < kTG; ++g) {
      const int gg = g0 + g < G ? g0 + g : g0;  // clamp: duplicates are never stored
      w[g] = u2d(pts[((long long)gg * nb + b) * pt_stride + ln]);
      wp[g] = w[g] * pinv;
    }
    const uint64_t* b0 = babies.c0[b];
    const uint64_t* b1 = babies.c1[b];
#pragma unroll
    for (int t = 0; t < kTI; ++t) {
      const int ii = i0 + t < ni ? i0 + t : i0;
      const double x0 = u2d(b0[(long long)ii * baby_stride + ln]);
      const double x1 = u2d(b1[(long long)ii * baby_stride + ln]);
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
  }
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

}  // namespace
}  // namespace hck

extern "C" int hck_bsgs_mac(const hck_context* ctx, int limbs, int inputs, int babies, int giants,
                            const uint64_t* const* baby_c0, const uint64_t* const* baby_c1,
                            int64_t baby_stride, const uint64_t* pts, int64_t pt_stride, uint64_t* res,
                            void* stream) {
  if (!ctx || !baby_c0 || !baby_c1 || !pts || !res) return HCK_ERR_ARG;
  if (limbs < 1 || limbs > ctx->L || inputs < 1 || babies < 1 || babies > hck::kMaxBabies || giants < 1)
    return HCK_ERR_ARG;
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
      res, bp, baby_stride, babies, inputs, giants, pts, pt_stride, limbs, units_per_limb, tiles_i, tiles_g,
      total_units, ctx->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}
