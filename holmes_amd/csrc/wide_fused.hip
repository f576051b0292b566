// Fused hybrid key switch on 64-bit words: the wide-prime path's counterpart of ksfused.hip.
//
// The same five-kernel schedule and workspace tile layout (tile_layout.hpp) as the FP64 kernels,
// with residues held as 64-bit words (every prime below 2^60, wide_fused_ok: the reference's 60/59-bit
// production chain).
// Arithmetic (every bound below needs 16p <= 2^64):
//  * transforms run lazily: a forward pass of four stages takes words below 8p, adds 2p per stage
//    (w_ct, no reduction) and subtracts 8p once at its end, so its outputs lie below 8p; inverse
//    (Harvey) butterflies take and return words below 2p; products by twiddles and conversion factors
//    use Shoup's companions, whose lazy result lies below 2p for any 64-bit input.  Workspace words
//    keep these lazy ranges;
//  * key products are Montgomery products x k 2^-64 (below 1.5p for x < 8p, k < p), summed lazily
//    below 2p and multiplied by 2^64 mod p (Shoup, canonical result) once per output;
//  * the base-conversion sums run on the int8 matrix cores with the wide digit tables (wide_dev.hpp:
//    wdigits takes a canonical residue, wfold returns one).
// Outputs are canonical.
//
//   K1 wf_intt_rows   sigma_g(d) (natural) --INTT rows-->                              T1 (workspace)
//   K2 wf_cols_mconv  T1 --INTT cols (N^-1 hinv folded)--> digits --ModUp sums (MFMA)--> NTT cols --> T2
//   K3 wf_rows_ip     P limbs: T2 --NTT rows--> x_j;  acc = sum_j x_j key_j --INTT rows--> ACCP
//                     (or every extended limb, ending in the extended basis)
//   K4 wf_cols_mconv  ACCP --INTT cols--> ModDown sums P -> Q --NTT cols--> T4
//   K5 wf_rows_ipq    Q limbs: acc as in K3 (d itself for the digit's own limb); T4 --NTT rows--> v;
//                     out = (acc - v) P^-1 (+ sigma_g(add)) (+ acc_in)
//
// Every intermediate is an exact residue, so the outputs equal those of the separate-launch wide
// kernels and of the CPU oracle (same centered fast base conversion).  Algorithm: EasyFHE's key switch
// for fhe.homo_rotate (F.cv_modup, F.cv_innerproduct_*, F.cv_moddown; bench/cmp/report.py:26-30).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "tile_layout.hpp"
#include "wide_dev.hpp"

namespace hck {
namespace {

using u64 = uint64_t;

constexpr int kT = 256;         // threads per workgroup
constexpr int kItems = 64;      // ciphertexts per launch (key pointers passed by value)
constexpr int kYStride = 272;   // LDS stride of one (source, column) run of 256 words
constexpr int kMItems = 3;      // targets per quarter-wave per conversion pass
constexpr int kMPass = 8 * kMItems;

struct WKeysF {
  const u64* k[kItems];
};
struct WGalF {
  int per_item;
  uint32_t uniform;
  uint32_t g[kItems];
};
__device__ __forceinline__ uint32_t gal_of(const WGalF& G, int b) { return G.per_item ? G.g[b] : G.uniform; }

// Cooley-Tukey (u, v) -> (u + w v, u - w v) without a reduction: w v lies below 2p (Shoup, for any
// 64-bit v), so each stage raises the bound by 2p.  A forward pass of four stages takes words below 8p
// to words below 16p (<= 2^64 for p < 2^60: wide_fused_ok) and subtracts 8p once at its end
// (w_fwd_end), so every forward pass's outputs, and the transform's, lie below 8p.
// Gentleman-Sande (u, v) -> (u + v, (u - v) w), inputs and outputs below 2p.  p2 = 2p.
__device__ __forceinline__ void w_ct(u64& u, u64& v, u64 w, u64 ws, u64 p, u64 p2) {
  const u64 a = u;
  const u64 y = mulshoup_lazy(v, w, ws, p);
  u = a + y;
  v = a - y + p2;
}
__device__ __forceinline__ void w_fwd_end(u64 (&x)[16], u64 p) {
  const u64 p8 = 8 * p;
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = x[k] >= p8 ? x[k] - p8 : x[k];
}
__device__ __forceinline__ void w_gs(u64& u, u64& v, u64 w, u64 ws, u64 p, u64 p2) {
  const u64 a = u, b = v, s = a + b;
  u = s >= p2 ? s - p2 : s;
  v = mulshoup_lazy(a - b + p2, w, ws, p);
}

// ----------------------------------------------------------------- column transforms (16-thread slots)
// Root indices as in ksfused.hip: stage l of a column pairs rows 128 >> l apart; layout A holds rows
// j + 16k (group k >> (4 - l)), layout B rows 16j + k (group (j << (l - 4)) + (k >> (8 - l))).
__device__ __forceinline__ void wcol_fwd_lo(u64 (&x)[16], const u64* __restrict__ tw, const u64* __restrict__ tws,
                                            u64 p) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const int wi = (1 << l) + (k >> (4 - l));
      w_ct(x[k], x[k + h], tw[wi], tws[wi], p, 2 * p);
    }
  }
  w_fwd_end(x, p);
}

__device__ __forceinline__ void wcol_fwd_hi(u64 (&x)[16], int j, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 4; l < 8; ++l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const int wi = (1 << l) + (j << (l - 4)) + (k >> (8 - l));
      w_ct(x[k], x[k + h], tw[wi], tws[wi], p, 2 * p);
    }
  }
  w_fwd_end(x, p);
}

__device__ __forceinline__ void wcol_inv_hi(u64 (&x)[16], int j, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 7; l >= 4; --l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const int wi = (1 << l) + (j << (l - 4)) + (k >> (8 - l));
      w_gs(x[k], x[k + h], tw[wi], tws[wi], p, 2 * p);
    }
  }
}

// inverse stages 3..1 on layout A, then stage 0 with its root, N^-1 and the conversion's hinv folded:
// n0 = N^-1 hinv, n1 = N^-1 psi_rev_inv[1] hinv (WideConv::inv_n0 / inv_n1); inputs below 2p
__device__ __forceinline__ void wcol_inv_lo(u64 (&x)[16], const u64* __restrict__ tw, const u64* __restrict__ tws,
                                            u64 n0, u64 n0s, u64 n1, u64 n1s, u64 p) {
#pragma unroll
  for (int l = 3; l >= 1; --l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const int wi = (1 << l) + (k >> (4 - l));
      w_gs(x[k], x[k + h], tw[wi], tws[wi], p, 2 * p);
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // canonical results (the conversion's digits need them)
    const u64 a = x[k], b = x[k + 8];
    x[k] = wcanon2(mulshoup_lazy(a + b, n0, n0s, p), p);
    x[k + 8] = wcanon2(mulshoup_lazy(a - b + 2 * p, n1, n1s, p), p);
  }
}

// ----------------------------------------------------------------- row transforms (256 threads)
// stage l of row b: layout A (words j + 16k) groups (b << (l - 8)) + (k >> (12 - l)); layout B
// (words 16j + k) groups (b << (l - 8)) + (j << (l - 12)) + (k >> (16 - l)).
// Each stage addresses its roots from one per-stage base (tw + base, constant offsets), so that the
// stages' root addresses cost a few registers when the compiler hoists them out of a digit loop.
__device__ __forceinline__ void wrow_fwd_lo(u64 (&x)[16], int b, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 8; l < 12; ++l) {
    const int h = 2048 >> l;
    const int base = (1 << l) + (b << (l - 8));
    const u64* __restrict__ t = tw + base;
    const u64* __restrict__ ts = tws + base;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      w_ct(x[k], x[k + h], t[k >> (12 - l)], ts[k >> (12 - l)], p, 2 * p);
    }
  }
  w_fwd_end(x, p);
}

__device__ __forceinline__ void wrow_fwd_hi(u64 (&x)[16], int b, int j, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 12; l < 16; ++l) {
    const int h = 32768 >> l;
    const int base = (1 << l) + (b << (l - 8)) + (j << (l - 12));
    const u64* __restrict__ t = tw + base;
    const u64* __restrict__ ts = tws + base;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      w_ct(x[k], x[k + h], t[k >> (16 - l)], ts[k >> (16 - l)], p, 2 * p);
    }
  }
  w_fwd_end(x, p);
}

__device__ __forceinline__ void wrow_inv_hi(u64 (&x)[16], int b, int j, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 15; l >= 12; --l) {
    const int h = 32768 >> l;
    const int base = (1 << l) + (b << (l - 8)) + (j << (l - 12));
    const u64* __restrict__ t = tw + base;
    const u64* __restrict__ ts = tws + base;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      w_gs(x[k], x[k + h], t[k >> (16 - l)], ts[k >> (16 - l)], p, 2 * p);
    }
  }
}

__device__ __forceinline__ void wrow_inv_lo(u64 (&x)[16], int b, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
#pragma unroll
  for (int l = 11; l >= 8; --l) {
    const int h = 2048 >> l;
    const int base = (1 << l) + (b << (l - 8));
    const u64* __restrict__ t = tw + base;
    const u64* __restrict__ ts = tws + base;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      w_gs(x[k], x[k + h], t[k >> (12 - l)], ts[k >> (12 - l)], p, 2 * p);
    }
  }
}

// NTT rows pass of row group g, x as load_t returns it (map T, layout A); returns layout A under map N
// (the thread's natural words nat_a(g) + 16k).
__device__ __forceinline__ void wrows_fwd_t(u64 (&x)[16], int g, u64* S, const u64* __restrict__ tw,
                                            const u64* __restrict__ tws, u64 p) {
  const RowMap mt = map_t(), mn = map_n();
  wrow_fwd_lo(x, g + 16 * mt.rb, tw, tws, p);
  row_xchg<true, false>(x, S, mt, mn);
  wrow_fwd_hi(x, g + 16 * mn.rb, mn.j, tw, tws, p);
  row_xchg<false, true>(x, S, mn, mn);
}

// INTT rows pass of row group g held in layout A under map N; stores the result to the workspace.
__device__ __forceinline__ void wrows_inv_to_t(u64 (&x)[16], u64* __restrict__ dst_t, int g, u64* S,
                                               const u64* __restrict__ tw, const u64* __restrict__ tws, u64 p) {
  const RowMap mt = map_t(), mn = map_n();
  row_xchg<true, false>(x, S, mn, mn);
  wrow_inv_hi(x, g + 16 * mn.rb, mn.j, tw, tws, p);
  row_xchg<false, true>(x, S, mn, mt);
  wrow_inv_lo(x, g + 16 * mt.rb, tw, tws, p);
#pragma unroll
  for (int k = 0; k < 16; ++k) dst_t[ws_a(g, k)] = x[k];
}

// ----------------------------------------------------------------- K1: INTT rows of d
// Limb i (< limbs) of item b reads input limb limb0 + i under prime prime0 + i and writes workspace limb
// i of a `limbs`-limb item.
__global__ __launch_bounds__(kT) void wf_intt_rows(const u64* __restrict__ d, long long d_stride, const WGalF G,
                                                   int limb0, int prime0, u64* __restrict__ t1, int limbs, int batch,
                                                   WideTables T) {
  __shared__ u64 S[kRowLds];
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= 16 * limbs) return;
  const int i = id.tile >> 4, rg = id.tile & 15, b = id.b, pi = prime0 + i;
  const u64 p = T.p[pi];
  u64 x[16];
  load_gal_raw(x, d + (long long)b * d_stride + (long long)(limb0 + i) * kN, nat_a(rg), gal_of(G, b));
  wrows_inv_to_t(x, t1 + ((long long)b * limbs + i) * kN, rg, S, T.inv + (size_t)pi * kN, T.inv_s + (size_t)pi * kN,
                 p);
}

// ----------------------------------------------------------------- K2 / K4: cols + conversion
// Block: columns (c0, c0 + 1) of conversion group y (a ModUp digit, or a ModDown component) of item z;
// 16 slots of 16 threads.  Phase 1: slot sigma = (source sigma >> 1, column sigma & 1) runs the INTT
// column stages of its source column and leaves the centered residue's digit word in run sigma of D.
// Phase 2 (as ksfused.hip's cols_mconv_body): wave w takes column w >> 1 and half w & 1 of each pass's
// 8 mi targets; quarter g owns mi (<= MI) of them, MFMA rows 4g + r; a lane supplies A row j (the
// digit bytes of sources 2g, 2g + 1 for target ta(j)) and B column j (the digit words of coefficient
// j + 16k), and receives rows 4g + r at column j: rows j + 16k of its targets over the 16 tiles, the
// forward column pass's layout A.  SEPX keeps separate exchange runs (X) so that D serves every pass.
struct WConvArgs {
  const u64* src;
  long long src_zs, src_ys;
  int src_off_y;
  u64* dst;
  long long dst_zs, dst_ys;
  const WideConv* cc_base;
  int cc_y;
  const u64* zsrc;  // RS: the extra source limb Z, group (z, y) at zsrc + z src_zs + y src_ys
};

// RS (the ModDown fused with the rescale, WideState::mdrs): after phase 1, slots 0 and 1 also run the
// INTT cols of Z, the q_{ell-1} limb of P * acc + IP (P^-1 folded into its last stage); phase 1c
// forms, for every coefficient of the two columns, the centered residue
// r = [Z P^-1 - sum_s ybar_s hmod[s][nt]]_{q_{ell-1}}, the q_{ell-1} limb of the ModDown output in
// the coefficient domain; phase 2 adds r to every stored target's sum (whose factors carry P^-1).
// With the finish of wf_rows_ipq_rs this gives ((IP - NTT(conv)) P^-1 + acc - NTT(r)) q_{ell-1}^-1,
// the ModDown followed by the rescale, exactly.
// MI: targets per quarter-wave per pass (kMItems, or 2 for conversions of at most 16 targets: 154
// instead of 206 VGPRs, three waves per SIMD).
template <bool SEPX, bool RS = false, int MI = kMItems>
__global__ __launch_bounds__(kT, 2) void wf_cols_mconv(const WConvArgs A, WideTables T, const wv4i* __restrict__ dig) {
  __shared__ u64 D[16 * kYStride];
  __shared__ u64 X[SEPX ? 16 * kYStride : 1];
  __shared__ long long Z[RS ? 2 * kYStride : 1];
  const int y = blockIdx.y;
  const long long z = blockIdx.z;
  const WideConv& C = A.cc_base[y * A.cc_y];
  const int ns = C.ns, nt = C.nt;
  const int t = threadIdx.x, sigma = t >> 4, j = t & 15;
  const int c0 = blockIdx.x * 2;
  // phase 1
  {
    const int s = sigma >> 1, cl = sigma & 1;
    const bool act = s < ns;
    const int sp = C.src_prime[act ? s : 0];
    const u64 p = T.p[sp];
    const u64* __restrict__ tw = T.inv + (size_t)sp * kN;
    const u64* __restrict__ tws = T.inv_s + (size_t)sp * kN;
    u64 x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = 0;
    if (act) {
      const u64* col = A.src + z * A.src_zs + y * A.src_ys + (long long)(y * A.src_off_y + s) * kN +
                       (long long)(c0 + cl) * 16;
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];  // rows 16 j + k: wpos = 4096 k + 16 c + j
      wcol_inv_hi(x, j, tw, tws, p);
    }
    u64* R = D + sigma * kYStride;
    col_b_to_a(x, R, j);
    if (act) wcol_inv_lo(x, tw, tws, C.inv_n0[s], C.inv_n0_s[s], C.inv_n1[s], C.inv_n1_s[s], p);
    // an idle source stores zero digits
#pragma unroll
    for (int k = 0; k < 16; ++k) R[j + 16 * k] = act ? wdigits(x[k], p) : 0ULL;
    if constexpr (RS) {
      if (sigma < 2) {  // phase 1b (one wave): Z P^-1 of column cl, canonical, into run cl of Z
        const int zp = C.dst_prime[nt];
        const u64 pz = T.p[zp];
        const u64* __restrict__ twz = T.inv + (size_t)zp * kN;
        const u64* __restrict__ twzs = T.inv_s + (size_t)zp * kN;
        const u64* col = A.zsrc + z * A.src_zs + y * A.src_ys + (long long)(c0 + cl) * 16;
#pragma unroll
        for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];
        wcol_inv_hi(x, j, twz, twzs, pz);
        u64* RZ = reinterpret_cast<u64*>(Z) + cl * kYStride;
        col_b_to_a(x, RZ, j);
        wcol_inv_lo(x, twz, twzs, C.z_n0, C.z_n0_s, C.z_n1, C.z_n1_s, pz);
#pragma unroll
        for (int k = 0; k < 16; ++k) RZ[j + 16 * k] = x[k];
      }
    }
  }
  __syncthreads();
  if constexpr (RS) {  // phase 1c: r for the 512 coefficients of the two columns, two per thread
    const u64 pz = T.p[C.dst_prime[nt]];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int q = t + 256 * u, cl = q >> 8, pos = q & 255;
      u64 acc = 0;
      for (int s = 0; s < ns; ++s) {  // ybar_s hmod[s][nt] with the sign of the centered digit word
        const long long yb = (long long)((D[(2 * s + cl) * kYStride + pos] ^ kDigitBias) - kDigitBias);
        const u64 m = wmulc(yb < 0 ? 0ULL - (u64)yb : (u64)yb, C.hmod[s][nt], C.hmod_s[s][nt], pz);
        acc = yb < 0 ? wsub(acc, m, pz) : wadd(acc, m, pz);
      }
      const u64 v = wsub((u64)Z[cl * kYStride + pos], acc, pz);
      Z[cl * kYStride + pos] = 2 * v > pz ? (long long)v - (long long)pz : (long long)v;
    }
    __syncthreads();
  }
  // phase 2
  const int w = t >> 6, g = (t >> 4) & 3;
  const int cl = w >> 1, h = w & 1;
  const u64* B0 = D + (4 * g + cl) * kYStride + j;      // source 2 g, column cl
  const u64* B1 = D + (4 * g + 2 + cl) * kYStride + j;  // source 2 g + 1
  u64* RX = (SEPX ? X : D) + sigma * kYStride;
  u64* dbase = A.dst + z * A.dst_zs + y * A.dst_ys + (long long)(c0 + cl) * 16;
  const wv4i* __restrict__ tab = dig + C.dig_off;
  for (int base = 0; base < nt;) {
    // mi targets per quarter in this pass (at most MI): the last pass spreads what is left over
    // every quarter, so that no wave idles while another folds three targets
    const int mi = min(MI, (nt - base + 7) / 8);
    // constants of MFMA row j: target of quarter j >> 2, item j & 3
    const int ta = base + (4 * h + (j >> 2)) * mi + (j & 3);
    const bool arow = (j & 3) < mi && ta < nt;
    wv4i av[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) av[c] = arow ? tab[((ta >> 4) * 8 + c) * 64 + 16 * g + (ta & 15)] : wv4i{0, 0, 0, 0};
    int to[MI], tp[MI], ts[MI];
    u64 pr[MI];
    double tinv[MI];
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      to[r] = r < mi ? base + (4 * h + g) * mi + r : nt;
      const int tt = to[r] < nt ? to[r] : 0;
      tp[r] = C.dst_prime[tt];
      ts[r] = C.dst_slot[tt];
      pr[r] = T.p[tp[r]];
      tinv[r] = C.fold_inv[tt];
    }
    u64 x[MI][16];
    uint64_t w0 = B0[0], w1 = B1[0];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const wv4i bv = {(int)(uint32_t)w0, (int)(uint32_t)(w0 >> 32), (int)(uint32_t)w1, (int)(uint32_t)(w1 >> 32)};
      wv4i acc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[c], bv, wv4i{0, 0, 0, 0}, 0, 0, 0);
      if (k < 15) {  // the next tile's digit words are read while this tile's sums are folded
        w0 = B0[16 * (k + 1)];
        w1 = B1[16 * (k + 1)];
      }
      const long long rz = RS ? Z[cl * kYStride + j + 16 * k] : 0;  // row j + 16k of column cl
#pragma unroll
      for (int r = 0; r < MI; ++r) {
        if constexpr (RS) x[r][k] = r < mi ? wfold_add(acc, r, pr[r], tinv[r], rz) : 0;
        else x[r][k] = r < mi ? wfold(acc, r, pr[r], tinv[r]) : 0;
        asm volatile("" : "+v"(x[r][k]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!SEPX) __syncthreads();  // every wave is done reading D before its runs become exchange buffers
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      if (r >= mi) break;  // uniform over the block
      const bool act = to[r] < nt;
      const u64* __restrict__ tw = T.fwd + (size_t)tp[r] * kN;
      const u64* __restrict__ tws = T.fwd_s + (size_t)tp[r] * kN;
      if (act) wcol_fwd_lo(x[r], tw, tws, pr[r]);
      col_a_to_b(x[r], RX, j);
      if (act) {
        wcol_fwd_hi(x[r], j, tw, tws, pr[r]);
        u64* col = dbase + (long long)ts[r] * kN;
#pragma unroll
        for (int k = 0; k < 16; ++k) col[4096 * k + j] = x[r][k];
      }
    }
    base += 8 * mi;
  }
}

// ----------------------------------------------------------------- inner product of one tile
// sb / sa = sum_j x_j key_j[comp] mod p over the digits j of item b, extended limb e (prime pi), row
// group rg: x_j the NTT rows pass of T2 digit j (below 8p), or, for the digit that holds limb e, d
// itself read through sigma_g.  Montgomery products summed below 2p, then one product by 2^64 mod p:
// canonical results.
struct WIp {
  const u64* d;
  long long d_stride;
  const u64* t2;
  const u64* key;
  int ell, beta, L, K, alpha, beta_max;
};

// FINISH = false leaves the sums in the Montgomery domain (x k 2^-64, below 2p) and INIT = false adds to
// them: the grouped kernel runs several items' inner products into one pair of sums.
template <bool INIT = true, bool FINISH = true>
__device__ __forceinline__ void wtile_ip(u64 (&sb)[16], u64 (&sa)[16], u64 (&x)[16], const WIp& I, int b, int e,
                                         int pi, int rg, uint32_t g, u64* S, const u64* __restrict__ tw,
                                         const u64* __restrict__ tws, const WideTables& T) {
  const u64 p = T.p[pi], p2 = 2 * p, mneg = T.mneg[pi];
  const int ext_l = I.ell + I.K;
  const long long comp = (long long)I.beta_max * (I.L + I.K) * kN;
  const int own = e < I.ell ? e / I.alpha : -1;
  const long long na = nat_a(rg);
  const u64* t2b = I.t2 + ((long long)b * I.beta * ext_l + e) * kN;
  // one key component at a time: the 16 words of the other are not live across the products
  auto mac = [&](u64 (&acc)[16], const u64* __restrict__ kp) {
    u64 kw[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) kw[k] = kp[16 * k];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const u64 v = acc[k] + wmont(x[k], kw[k], p, mneg);  // below 3.5p
      acc[k] = v >= p2 ? v - p2 : v;
    }
  };
  if constexpr (INIT) {
#pragma unroll
    for (int k = 0; k < 16; ++k) sb[k] = sa[k] = 0;
  }
  for (int jd = 0; jd < I.beta; ++jd) {
    if (jd == own) {
      load_gal_raw(x, I.d + (long long)b * I.d_stride + (long long)e * kN, na, g);
    } else {
      load_t(x, t2b + (long long)jd * ext_l * kN, rg);
      wrows_fwd_t(x, rg, S, tw, tws, p);
    }
    const u64* kp = I.key + ((long long)jd * (I.L + I.K) + pi) * kN + na;
    mac(sb, kp);
    mac(sa, kp + comp);
  }
  if constexpr (!FINISH) return;
  const u64 r = T.r64[pi], rs = T.r64_s[pi];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    sb[k] = wmulc(sb[k], r, rs, p);
    sa[k] = wmulc(sa[k], r, rs, p);
  }
}

// ----------------------------------------------------------------- K3: inner product, P limbs / ext
// Tile = (row group, extended limb e0 + tile / 16).  Without ext_b the kernel covers the K special
// limbs (e0 = ell) and runs the inner product's INTT rows pass into ACCP ([item][2][K], workspace
// layout) for the ModDown conversion.  With ext_b it covers every extended limb (e0 = 0) and ends the
// key switch in the extended basis: (P sigma(add) + IP_b, IP_a) (+ acc) over Q u P, natural layout.
__global__ __launch_bounds__(kT, 2) void wf_rows_ip(const WIp I, const WGalF G, WKeysF keys, int batch, int tiles,
                                                    int e0, u64* __restrict__ accp, const u64* __restrict__ add,
                                                    long long add_stride, u64* ext_b, u64* ext_a, long long ext_stride,
                                                    const u64* acc_b, const u64* acc_a, long long acc_stride,
                                                    WideTables T) {
  __shared__ u64 S[kRowLds];
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= tiles) return;
  const int b = id.b, e = e0 + (id.tile >> 4), rg = id.tile & 15;
  const uint32_t g = gal_of(G, b);
  const int pi = e < I.ell ? e : I.L + (e - I.ell);
  const u64 p = T.p[pi];
  WIp Ib = I;
  Ib.key = keys.k[b];
  u64 sb[16], sa[16], x[16];
  wtile_ip(sb, sa, x, Ib, b, e, pi, rg, g, S, T.fwd + (size_t)pi * kN, T.fwd_s + (size_t)pi * kN, T);
  const long long na = nat_a(rg);
  if (ext_b) {
    if (e < I.ell && add) {
      load_gal_raw(x, add + (long long)b * add_stride + (long long)e * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] = wadd(sb[k], wmulc(x[k], T.pmod[pi], T.pmod_s[pi], p), p);
    }
    if (acc_b) {
      // read before the store below by the same thread: ext may alias acc
      const u64* ab = acc_b + (long long)b * acc_stride + (long long)e * kN + na;
      const u64* aa = acc_a + (long long)b * acc_stride + (long long)e * kN + na;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        sb[k] = wadd(sb[k], ab[16 * k], p);
        sa[k] = wadd(sa[k], aa[16 * k], p);
      }
    }
    u64* ob = ext_b + (long long)b * ext_stride + (long long)e * kN + na;
    u64* oa = ext_a + (long long)b * ext_stride + (long long)e * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      ob[16 * k] = sb[k];
      oa[16 * k] = sa[k];
    }
    return;
  }
  // ACCP holds tiles / 16 limbs per component from e0 on: the K special limbs, or (ModDown fused with
  // the rescale, e0 = ell - 1) the q_{ell-1} limb first, as Z = IP + P (sigma(add) + acc)
  const int k1 = tiles >> 4;
  if (e < I.ell) {
    const u64 pm = T.pmod[pi], pms = T.pmod_s[pi];
    if (add) {
      load_gal_raw(x, add + (long long)b * add_stride + (long long)e * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] = wadd(sb[k], wmulc(x[k], pm, pms, p), p);
    }
    if (acc_b) {
      const u64* ab = acc_b + (long long)b * acc_stride + (long long)e * kN + na;
      const u64* aa = acc_a + (long long)b * acc_stride + (long long)e * kN + na;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        sb[k] = wadd(sb[k], wmulc(ab[16 * k], pm, pms, p), p);
        sa[k] = wadd(sa[k], wmulc(aa[16 * k], pm, pms, p), p);
      }
    }
  }
  u64* o = accp + ((long long)b * 2 * k1 + (e - e0)) * kN;
  const u64* twi = T.inv + (size_t)pi * kN;
  const u64* twis = T.inv_s + (size_t)pi * kN;
  wrows_inv_to_t(sb, o, rg, S, twi, twis, p);
  wrows_inv_to_t(sa, o + (long long)k1 * kN, rg, S, twi, twis, p);
}

// ----------------------------------------------------------------- K3 of grouped extended-basis rotations
// Output o (one tile of it per workgroup) is
//   acc[o] + sum_m (P sigma_m(add[b]) + IP_b(sigma_m(d[b])), IP_a(sigma_m(d[b])))   over b = m * outputs + o,
// each member with its own Galois element and key: the members' products and P sigma(add) (as the
// Montgomery product by P mod p) run into one pair of lazy sums, scaled by 2^64 mod p once, so the
// extended accumulator is read and written once per output.  Natural layout; ext may alias acc.
__global__ __launch_bounds__(kT, 2) void wf_rows_ip_sum(const WIp I, const WGalF G, WKeysF keys, int outputs, int group,
                                                        int tiles, const u64* __restrict__ add, long long add_stride,
                                                        u64* ext_b, u64* ext_a, long long ext_stride, const u64* acc_b,
                                                        const u64* acc_a, long long acc_stride, WideTables T) {
  __shared__ u64 S[kRowLds];
  const TileId id = decode_tile(outputs, blockIdx.x);
  if (id.tile >= tiles) return;
  const int o = id.b, e = id.tile >> 4, rg = id.tile & 15;
  const int pi = e < I.ell ? e : I.L + (e - I.ell);
  const u64 p = T.p[pi], p2 = 2 * p, mneg = T.mneg[pi];
  const u64* tw = T.fwd + (size_t)pi * kN;
  const u64* tws = T.fwd_s + (size_t)pi * kN;
  const long long na = nat_a(rg);
  u64 sb[16], sa[16], x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) sb[k] = sa[k] = 0;
  for (int m = 0; m < group; ++m) {
    const int b = m * outputs + o;
    const uint32_t g = gal_of(G, b);
    WIp Ib = I;
    Ib.key = keys.k[b];
    wtile_ip<false, false>(sb, sa, x, Ib, b, e, pi, rg, g, S, tw, tws, T);
    if (e < I.ell && add) {
      load_gal_raw(x, add + (long long)b * add_stride + (long long)e * kN, na, g);
      const u64 pm = T.pmod[pi];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const u64 v = sb[k] + wmont(x[k], pm, p, mneg);  // below 3.5p
        sb[k] = v >= p2 ? v - p2 : v;
      }
    }
  }
  const u64 r = T.r64[pi], rs = T.r64_s[pi];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    sb[k] = wmulc(sb[k], r, rs, p);
    sa[k] = wmulc(sa[k], r, rs, p);
  }
  if (acc_b) {
    // read before the store below by the same thread: ext may alias acc
    const u64* ab = acc_b + (long long)o * acc_stride + (long long)e * kN + na;
    const u64* aa = acc_a + (long long)o * acc_stride + (long long)e * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      sb[k] = wadd(sb[k], ab[16 * k], p);
      sa[k] = wadd(sa[k], aa[16 * k], p);
    }
  }
  u64* ob = ext_b + (long long)o * ext_stride + (long long)e * kN + na;
  u64* oa = ext_a + (long long)o * ext_stride + (long long)e * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    ob[16 * k] = sb[k];
    oa[16 * k] = sa[k];
  }
}

// ----------------------------------------------------------------- K5: Q limbs: inner product + ModDown
// out_b = (IP_b - v_b) P^-1 + sigma_g(add) (+ acc_b),  out_a = (IP_a - v_a) P^-1 (+ acc_a),
// v = the NTT rows pass of the ModDown conversion T4 ([item][2][ell], workspace layout; below 8p).
__global__ __launch_bounds__(kT, 2) void wf_rows_ipq(const WIp I, const WGalF G, WKeysF keys, int batch,
                                                     const u64* __restrict__ t4, const u64* __restrict__ add,
                                                     long long add_stride, const u64* __restrict__ acc_b,
                                                     const u64* __restrict__ acc_a, long long acc_stride,
                                                     u64* __restrict__ out_b, u64* __restrict__ out_a,
                                                     long long out_stride, WideTables T) {
  __shared__ u64 S[kRowLds];
  __shared__ u64 Park[16 * kT];  // sa while sb is finished (keeps both out of the registers at once)
  const int ell = I.ell;
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= 16 * ell) return;
  const int b = id.b, i = id.tile >> 4, rg = id.tile & 15;
  const uint32_t g = gal_of(G, b);
  const u64 p = T.p[i];
  const u64* tw = T.fwd + (size_t)i * kN;
  const u64* tws = T.fwd_s + (size_t)i * kN;
  WIp Ib = I;
  Ib.key = keys.k[b];
  u64 sb[16], sa[16], x[16];
  wtile_ip(sb, sa, x, Ib, b, i, i, rg, g, S, tw, tws, T);
  const long long na = nat_a(rg);
  const u64 pv = T.pinv[i], pvs = T.pinv_s[i];
  auto finish = [&](u64 (&s)[16], int comp, const u64* addend, const u64* ac, u64* out) {
    load_t(x, t4 + ((long long)b * 2 * ell + (long long)comp * ell + i) * kN, rg);
    wrows_fwd_t(x, rg, S, tw, tws, p);
#pragma unroll
    for (int k = 0; k < 16; ++k) s[k] = wcanon2(mulshoup_lazy(s[k] + 8 * p - x[k], pv, pvs, p), p);  // v < 8p
    if (addend) {
      load_gal_raw(x, addend + (long long)b * add_stride + (long long)i * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] = wadd(s[k], x[k], p);
    }
    if (ac) {
      const u64* a = ac + (long long)b * acc_stride + (long long)i * kN + na;
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] = wadd(s[k], a[16 * k], p);
    }
    u64* o = out + (long long)b * out_stride + (long long)i * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) o[16 * k] = s[k];
  };
#pragma unroll
  for (int k = 0; k < 16; ++k) Park[k * kT + threadIdx.x] = sa[k];
  finish(sb, 0, add, acc_b, out_b);
#pragma unroll
  for (int k = 0; k < 16; ++k) sa[k] = Park[k * kT + threadIdx.x];
  finish(sa, 1, nullptr, acc_a, out_a);
}

// ----------------------------------------------------------------- K5 of the ModDown fused with the rescale
// Q limbs i < ell - 1: out = (IP P^-1 - v + sigma_g(add) + acc) q_{ell-1}^-1, v the NTT rows pass of
// T4 = conv P^-1 + r ([item][2][ell - 1], workspace layout; below 8p), then the post-ops
// out <- (twice ? 2 out : out) - sub (+ scalar[i] on out_b).  With a0 .. b1 set the accumulators are
// the tensor terms a0 b0 and a0 b1 + a1 b0, formed here.
struct WRsPost {
  const u64 *sub_b, *sub_a;
  long long sub_stride;
  int twice, has_scalar;
  u64 scalar[kMaxPrimes];
  const u64 *a0, *a1, *b0, *b1;
  long long a_stride, b_stride;
  const u64 *ql, *ql_s;  // q_{ell-1}^-1 mod q_i and its companion at this level
};

__global__ __launch_bounds__(kT, 2) void wf_rows_ipq_rs(const WIp I, const WGalF G, WKeysF keys, int batch,
                                                        const u64* __restrict__ t4, const u64* __restrict__ add,
                                                        long long add_stride, const u64* __restrict__ acc_b,
                                                        const u64* __restrict__ acc_a, long long acc_stride,
                                                        u64* __restrict__ out_b, u64* __restrict__ out_a,
                                                        long long out_stride, const WRsPost post, WideTables T) {
  __shared__ u64 S[kRowLds];
  __shared__ u64 Park[16 * kT];  // sa while sb is finished
  const int nq = I.ell - 1;
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= 16 * nq) return;
  const int b = id.b, i = id.tile >> 4, rg = id.tile & 15;
  const uint32_t g = gal_of(G, b);
  const u64 p = T.p[i], mneg = T.mneg[i];
  const u64* tw = T.fwd + (size_t)i * kN;
  const u64* tws = T.fwd_s + (size_t)i * kN;
  WIp Ib = I;
  Ib.key = keys.k[b];
  u64 sb[16], sa[16], x[16];
  wtile_ip(sb, sa, x, Ib, b, i, i, rg, g, S, tw, tws, T);
  const long long na = nat_a(rg);
  const u64 pv = T.pinv[i], pvs = T.pinv_s[i], ql = post.ql[i], qls = post.ql_s[i];
  const u64 r64 = T.r64[i], r64s = T.r64_s[i];
  const bool prod = post.a0 != nullptr;
  const long long ao = (long long)b * post.a_stride + (long long)i * kN + na;
  const long long bo = (long long)b * post.b_stride + (long long)i * kN + na;
  const long long so = (long long)b * post.sub_stride + (long long)i * kN + na;
  // x1 y1 (+ x2 y2): Montgomery products of canonical words (each below 2p), one product by 2^64 mod p
  auto finish = [&](u64 (&s)[16], int comp, const u64* addend, const u64* ac, const u64* sub, u64 scal,
                    const u64* x1, const u64* y1, const u64* x2, const u64* y2, u64* out) {
    load_t(x, t4 + ((long long)b * 2 * nq + (long long)comp * nq + i) * kN, rg);
    wrows_fwd_t(x, rg, S, tw, tws, p);
#pragma unroll
    for (int k = 0; k < 16; ++k) s[k] = wmulc(s[k], pv, pvs, p) + 8 * p - x[k];  // below 9p
    if (x1) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        u64 m = wmont(x1[16 * k], y1[16 * k], p, mneg);
        if (x2) m += wmont(x2[16 * k], y2[16 * k], p, mneg);
        s[k] += wmulc(m, r64, r64s, p);  // below 10p
      }
    }
    if (addend) {
      load_gal_raw(x, addend + (long long)b * add_stride + (long long)i * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] += x[k];
    }
    if (ac) {
      const u64* a = ac + (long long)b * acc_stride + (long long)i * kN + na;
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] += a[16 * k];  // below 12p <= 2^64 (p < 2^60)
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      u64 r = wcanon2(mulshoup_lazy(s[k], ql, qls, p), p);
      if (post.twice) r = wadd(r, r, p);
      if (sub) r = wsub(r, sub[16 * k], p);
      s[k] = wadd(r, scal, p);
    }
    u64* o = out + (long long)b * out_stride + (long long)i * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) o[16 * k] = s[k];
  };
#pragma unroll
  for (int k = 0; k < 16; ++k) Park[k * kT + threadIdx.x] = sa[k];
  finish(sb, 0, add, prod ? nullptr : acc_b, post.sub_b ? post.sub_b + so : nullptr,
         post.has_scalar ? post.scalar[i] : 0, prod ? post.a0 + ao : nullptr, prod ? post.b0 + bo : nullptr, nullptr,
         nullptr, out_b);
#pragma unroll
  for (int k = 0; k < 16; ++k) sa[k] = Park[k * kT + threadIdx.x];
  finish(sa, 1, nullptr, prod ? nullptr : acc_a, post.sub_a ? post.sub_a + so : nullptr, 0,
         prod ? post.a0 + ao : nullptr, prod ? post.b1 + bo : nullptr, prod ? post.a1 + ao : nullptr,
         prod ? post.b0 + bo : nullptr, out_a);
}

// ----------------------------------------------------------------- ModDown / rescale finish
// Poly pl = blockIdx.x, limb i = blockIdx.z: v = NTT rows of T4[pl][i] (below 8p); out = (x - v) inv
// with x canonical (natural layout): inv = P^-1 (ModDown of an extended-basis input) or
// q_{ell-1}^-1 (rescale).  Grid (polys, 16, limbs).
__global__ __launch_bounds__(kT) void wf_rows_finish(const u64* __restrict__ t4, const u64* __restrict__ xq,
                                                     long long xq_stride, u64* __restrict__ out, long long out_stride,
                                                     int limbs, const u64* __restrict__ inv,
                                                     const u64* __restrict__ inv_s, WideTables T) {
  __shared__ u64 S[kRowLds];
  const int pl = blockIdx.x, rg = blockIdx.y, i = blockIdx.z;
  const u64 p = T.p[i];
  const long long na = nat_a(rg);
  u64 x[16], a[16];
  load_t(x, t4 + ((long long)pl * limbs + i) * kN, rg);
  load_gal_raw(a, xq + (long long)pl * xq_stride + (long long)i * kN, na, 1u);
  wrows_fwd_t(x, rg, S, T.fwd + (size_t)i * kN, T.fwd_s + (size_t)i * kN, p);
  const u64 w = inv[i], ws = inv_s[i];
  u64* o = out + (long long)pl * out_stride + (long long)i * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = wcanon2(mulshoup_lazy(a[k] + 8 * p - x[k], w, ws, p), p);
}

// ----------------------------------------------------------------- weighted sums with their rescale
// out[g] = rescale(sum_t w[t] x[g][t]) (+ add on the groups of add_mask), the combination never
// stored (hck_lincomb_rescale): wf_lc_intt_last forms the sum of the last limb and runs its INTT rows,
// the conversion lifts it to the lower primes, and wf_lc_finish forms each lower limb's sum again and
// finishes it with the NTT rows of the lift.  The sums are exact 128-bit sums of products of canonical
// words (each below p^2), folded once every kLcFold terms (a folded residue plus kLcFold - 1 products
// stays below p 2^64 for p < 2^60).
struct WLcRsArgs {
  const u64* x[kLcRsPtrs];  // group-major: x[g * terms + t]
  u64* out[kLcRsGroups];
  u64 add[kMaxPrimes];
  unsigned long long add_mask;
};
constexpr int kLcFold = 15;

// sum_t w[t][i] x[g][t] at limb i (prime pi) of row group rg's natural words na + 16 k, canonical
__device__ __forceinline__ void wlc_tile(u64 (&x)[16], const WLcRsArgs& A, int g, int terms,
                                         const u64* __restrict__ w, int wlimbs, int i, int pi, long long na,
                                         const WideTables& T) {
  const u64 p = T.p[pi], mneg = T.mneg[pi], r = T.r64[pi], rs = T.r64_s[pi];
  u128_t acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0;
  for (int t = 0; t < terms; ++t) {
    const u64* xs = A.x[g * terms + t] + (long long)i * kN + na;
    const u64 wt = w[(long long)t * wlimbs + i];
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] += (u128_t)xs[16 * k] * wt;
    if (t % kLcFold == kLcFold - 1 && t + 1 < terms) {  // uniform
#pragma unroll
      for (int k = 0; k < 16; ++k) acc[k] = wfold128(acc[k], p, mneg, r, rs);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = wfold128(acc[k], p, mneg, r, rs);
}

// Grid (16, groups): the last limb's sum, its INTT rows into the workspace layout
__global__ __launch_bounds__(kT) void wf_lc_intt_last(const WLcRsArgs A, int terms, const u64* __restrict__ w, int ell,
                                                      u64* __restrict__ tl, WideTables T) {
  __shared__ u64 S[kRowLds];
  const int rg = blockIdx.x, g = blockIdx.y, pi = ell - 1;
  u64 x[16];
  wlc_tile(x, A, g, terms, w, ell, pi, pi, nat_a(rg), T);
  wrows_inv_to_t(x, tl + (long long)g * kN, rg, S, T.inv + (size_t)pi * kN, T.inv_s + (size_t)pi * kN, T.p[pi]);
}

// Grid (groups, 16, ell - 1): out[g][i] = (sum_t w[t][i] x[g][t][i] - NTT rows(T4[g][i])) q_{ell-1}^-1
// (+ add[i]); the NTT rows pass leaves v below 8p
__global__ __launch_bounds__(kT) void wf_lc_finish(const WLcRsArgs A, int terms, const u64* __restrict__ w, int ell,
                                                   const u64* __restrict__ t4, const u64* __restrict__ inv,
                                                   const u64* __restrict__ inv_s, WideTables T) {
  __shared__ u64 S[kRowLds];
  const int g = blockIdx.x, rg = blockIdx.y, i = blockIdx.z, nt = ell - 1;
  const u64 p = T.p[i];
  const long long na = nat_a(rg);
  u64 x[16], a[16];
  load_t(x, t4 + ((long long)g * nt + i) * kN, rg);
  wlc_tile(a, A, g, terms, w, ell, i, i, na, T);
  wrows_fwd_t(x, rg, S, T.fwd + (size_t)i * kN, T.fwd_s + (size_t)i * kN, p);
  const u64 wv = inv[i], wvs = inv_s[i];
  const bool add = (A.add_mask >> g) & 1ull;  // uniform
  const u64 av = add ? A.add[i] : 0;
  u64* o = A.out[g] + (long long)i * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = wadd(wcanon2(mulshoup_lazy(a[k] + 8 * p - x[k], wv, wvs, p), p), av, p);
}

// ----------------------------------------------------------------- hoisted rotations
// The hoisted digits: digits[input][j][e] = the NTT-domain ModUp of digit j on extended limb e
// (canonical, natural layout; the digit's own limbs are the input's limbs).  Grid (16 (ell + K), beta,
// inputs): the row pass of each T2 tile, or a copy of the own limb.
__global__ __launch_bounds__(kT) void wf_hoist_store(const u64* __restrict__ t2, const u64* __restrict__ d,
                                                     long long d_stride, int ell, int beta, int alpha, int L, int K,
                                                     u64* __restrict__ digits, WideTables T) {
  __shared__ u64 S[kRowLds];
  const int e = blockIdx.x >> 4, rg = blockIdx.x & 15, j = blockIdx.y, b = blockIdx.z;
  const int ext_l = ell + K;
  const long long na = nat_a(rg);
  const long long off = ((long long)(b * beta + j) * ext_l + e) * kN;
  u64 x[16];
  if (e < ell && e / alpha == j) {
    load_gal_raw(x, d + (long long)b * d_stride + (long long)e * kN, na, 1u);
  } else {
    const int pi = e < ell ? e : L + (e - ell);
    const u64 p = T.p[pi];
    load_t(x, t2 + off, rg);
    wrows_fwd_t(x, rg, S, T.fwd + (size_t)pi * kN, T.fwd_s + (size_t)pi * kN, p);
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = wcanon8(x[k], p);
  }
  u64* o = digits + off + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = x[k];
}

// Item b rotates input (src0 + b) % inputs by its Galois element: the inner product reads every digit
// through sigma_g (ModUp commutes with sigma_g), with no row transform.  Montgomery products summed
// below 2p, then one product by 2^64 mod p: canonical.
struct WHoist {
  const u64* digits;
  int inputs, src0;
};
__device__ __forceinline__ void wtile_ip_h(u64 (&sb)[16], u64 (&sa)[16], u64 (&x)[16], const WHoist& H,
                                           const u64* __restrict__ key, int beta, int ell, int L, int K, int beta_max,
                                           int b, int e, int pi, int rg, uint32_t g, const WideTables& T) {
  const u64 p = T.p[pi], p2 = 2 * p, mneg = T.mneg[pi];
  const int ext_l = ell + K, src = (H.src0 + b) % H.inputs;
  const long long comp = (long long)beta_max * (L + K) * kN;
  const long long na = nat_a(rg);
  auto mac = [&](u64 (&acc)[16], const u64* __restrict__ kp) {
    u64 kw[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) kw[k] = kp[16 * k];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const u64 v = acc[k] + wmont(x[k], kw[k], p, mneg);
      acc[k] = v >= p2 ? v - p2 : v;
    }
  };
#pragma unroll
  for (int k = 0; k < 16; ++k) sb[k] = sa[k] = 0;
  for (int jd = 0; jd < beta; ++jd) {
    load_gal_raw(x, H.digits + ((long long)(src * beta + jd) * ext_l + e) * kN, na, g);
    const u64* kp = key + ((long long)jd * (L + K) + pi) * kN + na;
    mac(sb, kp);
    mac(sa, kp + comp);
  }
  const u64 r = T.r64[pi], rs = T.r64_s[pi];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    sb[k] = wmulc(sb[k], r, rs, p);
    sa[k] = wmulc(sa[k], r, rs, p);
  }
}

// P limbs of hoisted rotations: the inner product's INTT rows pass into ACCP ([item][2][K]).
__global__ __launch_bounds__(kT, 2) void wf_rows_ip_h(const WGalF G, WKeysF keys, int ell, int beta, int L, int K,
                                                      int beta_max, int batch, u64* __restrict__ accp, WHoist H,
                                                      WideTables T) {
  __shared__ u64 S[kRowLds];
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= 16 * K) return;
  const int b = id.b, e = ell + (id.tile >> 4), rg = id.tile & 15, pi = L + (e - ell);
  const u64 p = T.p[pi];
  u64 sb[16], sa[16], x[16];
  wtile_ip_h(sb, sa, x, H, keys.k[b], beta, ell, L, K, beta_max, b, e, pi, rg, gal_of(G, b), T);
  u64* o = accp + ((long long)b * 2 * K + (e - ell)) * kN;
  const u64* twi = T.inv + (size_t)pi * kN;
  const u64* twis = T.inv_s + (size_t)pi * kN;
  wrows_inv_to_t(sb, o, rg, S, twi, twis, p);
  wrows_inv_to_t(sa, o + (long long)K * kN, rg, S, twi, twis, p);
}

// Q limbs of hoisted rotations: out_b = (IP_b - v_b) P^-1 + sigma_g(c0 of the input), out_a = (IP_a - v_a) P^-1.
__global__ __launch_bounds__(kT, 2) void wf_rows_ipq_h(const WGalF G, WKeysF keys, int ell, int beta, int L, int K,
                                                       int beta_max, int batch, const u64* __restrict__ t4,
                                                       const u64* __restrict__ c0, long long c0_stride,
                                                       u64* __restrict__ out_b, u64* __restrict__ out_a,
                                                       long long out_stride, WHoist H, WideTables T) {
  __shared__ u64 S[kRowLds];
  __shared__ u64 Park[16 * kT];
  const TileId id = decode_tile(batch, blockIdx.x);
  if (id.tile >= 16 * ell) return;
  const int b = id.b, i = id.tile >> 4, rg = id.tile & 15;
  const uint32_t g = gal_of(G, b);
  const u64 p = T.p[i];
  const u64* tw = T.fwd + (size_t)i * kN;
  const u64* tws = T.fwd_s + (size_t)i * kN;
  u64 sb[16], sa[16], x[16];
  wtile_ip_h(sb, sa, x, H, keys.k[b], beta, ell, L, K, beta_max, b, i, i, rg, g, T);
  const long long na = nat_a(rg);
  const u64 pv = T.pinv[i], pvs = T.pinv_s[i];
  const int src = (H.src0 + b) % H.inputs;
  auto finish = [&](u64 (&s)[16], int comp, const u64* addend, u64* out) {
    load_t(x, t4 + ((long long)b * 2 * ell + (long long)comp * ell + i) * kN, rg);
    wrows_fwd_t(x, rg, S, tw, tws, p);
#pragma unroll
    for (int k = 0; k < 16; ++k) s[k] = wcanon2(mulshoup_lazy(s[k] + 8 * p - x[k], pv, pvs, p), p);
    if (addend) {
      load_gal_raw(x, addend + (long long)src * c0_stride + (long long)i * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) s[k] = wadd(s[k], x[k], p);
    }
    u64* o = out + (long long)b * out_stride + (long long)i * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) o[16 * k] = s[k];
  };
#pragma unroll
  for (int k = 0; k < 16; ++k) Park[k * kT + threadIdx.x] = sa[k];
  finish(sb, 0, c0, out_b);
#pragma unroll
  for (int k = 0; k < 16; ++k) sa[k] = Park[k * kT + threadIdx.x];
  finish(sa, 1, nullptr, out_a);
}

void launch_wconv_fused(const WConvArgs& A, int nt_max, dim3 grid, const WideState& W, hipStream_t s) {
  auto k = nt_max <= 16 ? wf_cols_mconv<false, false, 2> : nt_max <= kMPass ? wf_cols_mconv<false> : wf_cols_mconv<true>;
  k<<<grid, kT, 0, s>>>(A, W.t, (const wv4i*)W.conv_dig);
}

void launch_wconv_rs(const WConvArgs& A, int nt_max, dim3 grid, const WideState& W, hipStream_t s) {
  auto k = nt_max <= 16 ? wf_cols_mconv<false, true, 2>
                        : nt_max <= kMPass ? wf_cols_mconv<false, true> : wf_cols_mconv<true, true>;
  k<<<grid, kT, 0, s>>>(A, W.t, (const wv4i*)W.conv_dig);
}

}  // namespace

bool wide_fused_ok(const hck_context* c) {
  return c->wide && c->conv_engine == 1 && c->wide->conv_dig && c->wide->primes_below_2_60 && c->alpha <= kMaxAlpha &&
         c->K <= kMaxSpecial;
}

size_t wide_fused_bytes(const hck_context* c, int ell, int batch) {
  const size_t nb = (size_t)std::min(batch, kItems), beta = beta_of(c, ell), ext_l = (size_t)(ell + c->K);
  return nb * kN * 8 * (2 * (size_t)ell + beta * ext_l + 2 * (size_t)c->K);
}

int wide_ks_fused(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
                  const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
                  const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a,
                  long long out_stride, char* ws, hipStream_t s, uint64_t* ext_b, uint64_t* ext_a,
                  long long ext_stride, const uint32_t* galois_items) {
  if (!wide_fused_ok(c)) return HCK_ERR_UNSUPPORTED;
  const WideState& W = *c->wide;
  const int K = c->K, L = c->L, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN;
  const int last_digit = ell - alpha * (beta - 1);
  for (int b0 = 0; b0 < batch; b0 += kItems) {
    const int nb = std::min(kItems, batch - b0);
    WGalF G{};
    G.per_item = galois_items ? 1 : 0;
    G.uniform = galois;
    if (galois_items)
      for (int b = 0; b < nb; ++b) G.g[b] = galois_items[b0 + b];
    WKeysF kp{};
    for (int b = 0; b < nb; ++b) kp.k[b] = ksk[b0 + b];
    const uint64_t* dd = d + (long long)b0 * d_stride;
    const uint64_t* a0 = add ? add + (long long)b0 * add_stride : nullptr;
    u64* r1 = (u64*)ws;  // T1 [nb][ell], later T4 [nb][2][ell]
    u64* t2 = r1 + (long long)nb * 2 * ell * n;
    u64* accp = t2 + (long long)nb * beta * ext_l * n;
    const WIp I{dd, d_stride, t2, nullptr, ell, beta, L, K, alpha, bmax};
    // K1
    wf_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * nb), kT, 0, s>>>(dd, d_stride, G, 0, 0, r1, ell, nb,
                                                                                  W.t);
    HCK_CHECK_LAUNCH();
    // K2: ModUp, one block per (column pair, digit, item)
    launch_wconv_fused(WConvArgs{r1, (long long)ell * n, 0, alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                                 W.modup + (size_t)ell * bmax, 1},
                       ext_l - last_digit, dim3(128, beta, nb), W, s);
    HCK_CHECK_LAUNCH();
    if (ext_b) {
      const int tiles = 16 * ext_l, groups = (tiles + kXcds - 1) / kXcds;
      const long long ai = (long long)b0 * acc_stride, ei = (long long)b0 * ext_stride;
      wf_rows_ip<<<dim3(groups * kXcds * nb), kT, 0, s>>>(I, G, kp, nb, tiles, 0, nullptr, a0, add_stride, ext_b + ei,
                                                          ext_a + ei, ext_stride, acc_b ? acc_b + ai : nullptr,
                                                          acc_a ? acc_a + ai : nullptr, acc_stride, W.t);
      HCK_CHECK_LAUNCH();
      continue;
    }
    // K3 over the K special limbs
    {
      const int tiles = 16 * K, groups = (tiles + kXcds - 1) / kXcds;
      wf_rows_ip<<<dim3(groups * kXcds * nb), kT, 0, s>>>(I, G, kp, nb, tiles, ell, accp, nullptr, 0, nullptr, nullptr,
                                                          0, nullptr, nullptr, 0, W.t);
      HCK_CHECK_LAUNCH();
    }
    // K4: ModDown conversion, one block per (column pair, component, item); T4 reuses R1
    u64* t4 = r1;
    launch_wconv_fused(WConvArgs{accp, 2LL * K * n, (long long)K * n, 0, t4, 2LL * ell * n, (long long)ell * n,
                                 W.moddown + ell, 0},
                       ell, dim3(128, 2, nb), W, s);
    HCK_CHECK_LAUNCH();
    // K5: Q limbs
    {
      const int tiles = 16 * ell, groups = (tiles + kXcds - 1) / kXcds;
      const long long ai = (long long)b0 * acc_stride, oi = (long long)b0 * out_stride;
      wf_rows_ipq<<<dim3(groups * kXcds * nb), kT, 0, s>>>(I, G, kp, nb, t4, a0, add_stride,
                                                           acc_b ? acc_b + ai : nullptr, acc_a ? acc_a + ai : nullptr,
                                                           acc_stride, out_b + oi, out_a + oi, out_stride, W.t);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

// Workspace per item: R1 = T1 / T4 [2 ell limbs], T2 [beta (ell + K)], ACCP [2 (K + 1)].
size_t wide_fused_rs_bytes(const hck_context* c, int ell, int batch) {
  const size_t nb = (size_t)std::min(batch, kItems), beta = beta_of(c, ell), ext_l = (size_t)(ell + c->K);
  return nb * kN * 8 * (2 * (size_t)ell + beta * ext_l + 2 * (size_t)(c->K + 1));
}

// The key switch with its ModDown fused with the rescale (ks_rescaled on the wide path): K1, K2 as in
// wide_ks_fused; K3 over q_{ell-1} and the special limbs (Z and the P limbs into ACCP); K4 the
// ModDown-rescale conversion to q_0 .. q_{ell-2} (T4); K5 the Q limbs below ell - 1 with the post-ops.
int wide_ks_rescaled(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride,
                     uint32_t galois, const uint64_t* const* ksk, const uint64_t* add, long long add_stride,
                     const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride, uint64_t* out_b,
                     uint64_t* out_a, long long out_stride, char* ws, hipStream_t s, int twice,
                     const uint64_t* sub_b, const uint64_t* sub_a, long long sub_stride, const uint64_t* scalar,
                     const uint64_t* const* prod_ab, long long a_stride, long long b_stride) {
  if (!wide_fused_ok(c) || ell < 2) return HCK_ERR_UNSUPPORTED;
  if (batch < 1 || (acc_b == nullptr) != (acc_a == nullptr) || (sub_b == nullptr) != (sub_a == nullptr))
    return HCK_ERR_ARG;
  const WideState& W = *c->wide;
  const int K = c->K, L = c->L, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const int nq = ell - 1;
  const long long n = kN;
  const int last_digit = ell - alpha * (beta - 1);
  WRsPost post{};
  post.twice = twice;
  post.has_scalar = scalar != nullptr;
  for (int i = 0; scalar && i < nq; ++i) post.scalar[i] = scalar[i];
  post.ql = W.qlast_inv + (size_t)ell * L;
  post.ql_s = W.qlast_inv_s + (size_t)ell * L;
  for (int b0 = 0; b0 < batch; b0 += kItems) {
    const int nb = std::min(kItems, batch - b0);
    WGalF G{};
    G.uniform = galois;
    WKeysF kp{};
    for (int b = 0; b < nb; ++b) kp.k[b] = ksk[b0 + b];
    const uint64_t* dd = d + (long long)b0 * d_stride;
    const uint64_t* a0 = add ? add + (long long)b0 * add_stride : nullptr;
    const long long ai = (long long)b0 * acc_stride, oi = (long long)b0 * out_stride;
    const uint64_t* ab = acc_b ? acc_b + ai : nullptr;
    const uint64_t* aa = acc_a ? acc_a + ai : nullptr;
    post.sub_b = sub_b ? sub_b + (long long)b0 * sub_stride : nullptr;
    post.sub_a = sub_a ? sub_a + (long long)b0 * sub_stride : nullptr;
    post.sub_stride = sub_stride;
    if (prod_ab) {
      post.a0 = prod_ab[0] + (long long)b0 * a_stride;
      post.a1 = prod_ab[1] + (long long)b0 * a_stride;
      post.b0 = prod_ab[2] + (long long)b0 * b_stride;
      post.b1 = prod_ab[3] + (long long)b0 * b_stride;
      post.a_stride = a_stride;
      post.b_stride = b_stride;
    }
    u64* r1 = (u64*)ws;  // T1 [nb][ell], later T4 [nb][2][ell - 1]
    u64* t2 = r1 + (long long)nb * 2 * ell * n;
    u64* accp = t2 + (long long)nb * beta * ext_l * n;  // [nb][2][K + 1]: q_{ell-1}, then P
    const WIp I{dd, d_stride, t2, nullptr, ell, beta, L, K, alpha, bmax};
    // K1, K2 as in wide_ks_fused
    wf_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * nb), kT, 0, s>>>(dd, d_stride, G, 0, 0, r1, ell, nb,
                                                                                  W.t);
    HCK_CHECK_LAUNCH();
    launch_wconv_fused(WConvArgs{r1, (long long)ell * n, 0, alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                                 W.modup + (size_t)ell * bmax, 1},
                       ext_l - last_digit, dim3(128, beta, nb), W, s);
    HCK_CHECK_LAUNCH();
    // K3 over q_{ell-1} and the K special limbs
    {
      const int tiles = 16 * (K + 1), groups = (tiles + kXcds - 1) / kXcds;
      wf_rows_ip<<<dim3(groups * kXcds * nb), kT, 0, s>>>(I, G, kp, nb, tiles, ell - 1, accp, a0, add_stride, nullptr,
                                                          nullptr, 0, ab, aa, acc_stride, W.t);
      HCK_CHECK_LAUNCH();
    }
    // K4: the ModDown-rescale conversion, one block per (column pair, component, item); T4 reuses R1
    u64* t4 = r1;
    launch_wconv_rs(WConvArgs{accp + n, 2LL * (K + 1) * n, (long long)(K + 1) * n, 0, t4, 2LL * nq * n, (long long)nq * n,
                              W.mdrs + ell, 0, accp},
                    nq, dim3(128, 2, nb), W, s);
    HCK_CHECK_LAUNCH();
    // K5: Q limbs 0 .. ell - 2
    {
      const int tiles = 16 * nq, groups = (tiles + kXcds - 1) / kXcds;
      wf_rows_ipq_rs<<<dim3(groups * kXcds * nb), kT, 0, s>>>(I, G, kp, nb, t4, a0, add_stride, ab, aa, acc_stride,
                                                              out_b + oi, out_a + oi, out_stride, post, W.t);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

// Grouped extended-basis rotations (ks_fused_sum on the wide path): item b = m * outputs + o of d / add
// (Galois element galois_items[b], key ksk[b]) is member m of output o; K1 and K2 run over every item,
// as in wide_ks_fused, then wf_rows_ip_sum; workspace wide_fused_bytes(c, ell, outputs * group).
int wide_ks_fused_sum(const hck_context* c, int ell, int outputs, int group, const uint64_t* d, long long d_stride,
                      const uint32_t* galois_items, const uint64_t* const* ksk, const uint64_t* add,
                      long long add_stride, const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride,
                      uint64_t* ext_b, uint64_t* ext_a, long long ext_stride, char* ws, hipStream_t s) {
  const int batch = outputs * group;
  if (!wide_fused_ok(c)) return HCK_ERR_UNSUPPORTED;
  if (outputs < 1 || group < 1 || batch > kItems || (acc_b == nullptr) != (acc_a == nullptr)) return HCK_ERR_ARG;
  const WideState& W = *c->wide;
  const int K = c->K, L = c->L, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN;
  const int last_digit = ell - alpha * (beta - 1);
  WGalF G{};
  G.per_item = 1;
  WKeysF kp{};
  for (int b = 0; b < batch; ++b) {
    G.g[b] = galois_items[b];
    kp.k[b] = ksk[b];
  }
  u64* r1 = (u64*)ws;  // T1 [batch][ell]
  u64* t2 = r1 + (long long)batch * 2 * ell * n;
  const WIp I{d, d_stride, t2, nullptr, ell, beta, L, K, alpha, bmax};
  wf_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * batch), kT, 0, s>>>(d, d_stride, G, 0, 0, r1, ell,
                                                                                    batch, W.t);
  HCK_CHECK_LAUNCH();
  launch_wconv_fused(WConvArgs{r1, (long long)ell * n, 0, alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                               W.modup + (size_t)ell * bmax, 1},
                     ext_l - last_digit, dim3(128, beta, batch), W, s);
  HCK_CHECK_LAUNCH();
  const int tiles = 16 * ext_l, groups = (tiles + kXcds - 1) / kXcds;
  wf_rows_ip_sum<<<dim3(groups * kXcds * outputs), kT, 0, s>>>(I, G, kp, outputs, group, tiles, add, add_stride, ext_b,
                                                               ext_a, ext_stride, acc_b, acc_a, acc_stride, W.t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t wide_fused_rescale_bytes(const hck_context* c, int ell, int polys) {
  (void)c;
  return (size_t)polys * kN * 8 * (size_t)ell;  // TL [1] + T4 [ell - 1] per poly
}

// Rescale by q_{ell-1}: INTT rows of the last limb, the lift to the ell - 1 lower primes in the
// conversion kernel (INTT cols, centered residue, NTT cols), then the finish with q_{ell-1}^-1.
int wide_rescale_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride,
                       uint64_t* out, long long out_stride, char* ws, hipStream_t s) {
  const WideState& W = *c->wide;
  const long long n = kN;
  const int nt = ell - 1;
  u64* tl = (u64*)ws;                   // [polys][1]
  u64* t4 = tl + (long long)polys * n;  // [polys][ell - 1]
  WGalF G{};
  G.uniform = 1u;
  for (int p0 = 0; p0 < polys; p0 += 65535) {
    const int np = std::min(65535, polys - p0);
    wf_intt_rows<<<dim3(((16 + kXcds - 1) / kXcds) * kXcds * np), kT, 0, s>>>(
        in + (long long)p0 * in_stride, in_stride, G, ell - 1, ell - 1, tl + (long long)p0 * n, 1, np, W.t);
    HCK_CHECK_LAUNCH();
    launch_wconv_fused(WConvArgs{tl + (long long)p0 * n, n, 0, 0, t4 + (long long)p0 * nt * n, (long long)nt * n, 0,
                                 W.rescale + ell, 0},
                       nt, dim3(128, 1, np), W, s);
    HCK_CHECK_LAUNCH();
    const size_t lv = (size_t)ell * c->L;
    wf_rows_finish<<<dim3(np, 16, nt), kT, 0, s>>>(t4 + (long long)p0 * nt * n, in + (long long)p0 * in_stride,
                                                   in_stride, out + (long long)p0 * out_stride, out_stride, nt,
                                                   W.qlast_inv + lv, W.qlast_inv_s + lv, W.t);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

// hck_lincomb_rescale on the fused kernels (the weighted sums are formed where they are used);
// workspace wide_fused_rescale_bytes(c, ell, groups)
int wide_lincomb_rescale_fused(const hck_context* c, int ell, int groups, int terms, const uint64_t* const* x,
                               const uint64_t* w, uint64_t* const* out, const uint64_t* add, uint64_t add_mask,
                               char* ws, hipStream_t s) {
  if (groups < 1) return HCK_OK;
  if (ell < 2 || groups > kLcRsGroups || terms < 1 || (long long)groups * terms > kLcRsPtrs || !w) return HCK_ERR_ARG;
  const WideState& W = *c->wide;
  const long long n = kN;
  const int nt = ell - 1;
  u64* tl = (u64*)ws;                    // [groups][1]
  u64* t4 = tl + (long long)groups * n;  // [groups][ell - 1]
  WLcRsArgs A{};
  for (int j = 0; j < groups * terms; ++j) A.x[j] = x[j];
  for (int g = 0; g < groups; ++g) A.out[g] = out[g];
  if (add)
    for (int i = 0; i < nt; ++i) A.add[i] = add[i];
  A.add_mask = add ? add_mask : 0ull;
  wf_lc_intt_last<<<dim3(16, groups), kT, 0, s>>>(A, terms, w, ell, tl, W.t);
  HCK_CHECK_LAUNCH();
  launch_wconv_fused(WConvArgs{tl, n, 0, 0, t4, (long long)nt * n, 0, W.rescale + ell, 0}, nt, dim3(128, 1, groups), W, s);
  HCK_CHECK_LAUNCH();
  const size_t lv = (size_t)ell * c->L;
  wf_lc_finish<<<dim3(groups, 16, nt), kT, 0, s>>>(A, terms, w, ell, t4, W.qlast_inv + lv, W.qlast_inv_s + lv, W.t);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t wide_fused_moddown_bytes(const hck_context* c, int ell, int polys) {
  return (size_t)polys * kN * 8 * (size_t)(c->K + ell);  // TP [K] + T4 [ell] per poly
}

// ModDown of extended-basis polys ([ell + K] canonical limbs, Q first): INTT rows of the P limbs, the
// conversion P -> Q (INTT cols, sums, NTT cols), then the finish with P^-1.
int wide_moddown_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride,
                       uint64_t* out, long long out_stride, char* ws, hipStream_t s) {
  const WideState& W = *c->wide;
  const int K = c->K;
  const long long n = kN;
  u64* tp = (u64*)ws;                        // [polys][K]
  u64* t4 = tp + (long long)polys * K * n;  // [polys][ell]
  WGalF G{};
  G.uniform = 1u;
  for (int p0 = 0; p0 < polys; p0 += 65535) {
    const int np = std::min(65535, polys - p0);
    wf_intt_rows<<<dim3(((16 * K + kXcds - 1) / kXcds) * kXcds * np), kT, 0, s>>>(
        in + (long long)p0 * in_stride, in_stride, G, ell, c->L, tp + (long long)p0 * K * n, K, np, W.t);
    HCK_CHECK_LAUNCH();
    launch_wconv_fused(WConvArgs{tp + (long long)p0 * K * n, (long long)K * n, 0, 0, t4 + (long long)p0 * ell * n,
                                 (long long)ell * n, 0, W.moddown + ell, 0},
                       ell, dim3(128, 1, np), W, s);
    HCK_CHECK_LAUNCH();
    wf_rows_finish<<<dim3(np, 16, ell), kT, 0, s>>>(t4 + (long long)p0 * ell * n, in + (long long)p0 * in_stride,
                                                    in_stride, out + (long long)p0 * out_stride, out_stride, ell,
                                                    W.t.pinv, W.t.pinv_s, W.t);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

size_t wide_fused_hoist_bytes(const hck_context* c, int ell, int inputs) {
  const size_t nb = (size_t)std::min(inputs, kItems), beta = beta_of(c, ell), ext_l = (size_t)(ell + c->K);
  return nb * kN * 8 * ((size_t)ell + beta * ext_l);  // T1 [ell] + T2 [beta][ell + K] per input
}

// The hoisted digits of every input (wf_hoist_store's format): INTT rows, the ModUp conversion, then
// the row pass of every T2 tile stored canonical in the natural layout.
int wide_hoist_fused(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride,
                     uint64_t* digits, char* ws, hipStream_t s) {
  const WideState& W = *c->wide;
  const int K = c->K, alpha = c->alpha, beta = beta_of(c, ell), ext_l = ell + K, bmax = c->beta_max;
  const long long n = kN;
  const int last_digit = ell - alpha * (beta - 1);
  const int per = std::min(inputs, kItems);
  u64* t1 = (u64*)ws;
  u64* t2 = t1 + (long long)per * ell * n;
  WGalF G{};
  G.uniform = 1u;
  for (int b0 = 0; b0 < inputs; b0 += kItems) {
    const int nb = std::min(kItems, inputs - b0);
    const uint64_t* dd = d + (long long)b0 * d_stride;
    wf_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * nb), kT, 0, s>>>(dd, d_stride, G, 0, 0, t1, ell, nb,
                                                                                  W.t);
    HCK_CHECK_LAUNCH();
    launch_wconv_fused(WConvArgs{t1, (long long)ell * n, 0, alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                                 W.modup + (size_t)ell * bmax, 1},
                       ext_l - last_digit, dim3(128, beta, nb), W, s);
    HCK_CHECK_LAUNCH();
    wf_hoist_store<<<dim3(16 * ext_l, beta, nb), kT, 0, s>>>(t2, dd, d_stride, ell, beta, alpha, c->L, K,
                                                             digits + (long long)b0 * beta * ext_l * n, W.t);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

size_t wide_fused_hoisted_bytes(const hck_context* c, int ell, int items) {
  const size_t nb = (size_t)std::min(items, kItems);
  return nb * kN * 8 * (2 * (size_t)ell + 2 * (size_t)c->K);  // T4 [2][ell] + ACCP [2][K] per item
}

// Item i (< items) = rotation of input i % inputs by galois[i] with key ksk[i], from its hoisted digits:
// (sigma(c0) + KS_b(sigma(c1)), KS_a(sigma(c1))), the residues of wide_ks_fused with that element.
int wide_hoisted_fused(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
                       const uint64_t* const* ksk, const uint64_t* c0, long long in_stride, const uint64_t* digits,
                       uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws, hipStream_t s) {
  const WideState& W = *c->wide;
  const int K = c->K, L = c->L, beta = beta_of(c, ell), bmax = c->beta_max;
  const long long n = kN;
  for (int i0 = 0; i0 < items; i0 += kItems) {
    const int nb = std::min(kItems, items - i0);
    WGalF G{};
    G.per_item = 1;
    WKeysF kp{};
    for (int b = 0; b < nb; ++b) {
      G.g[b] = galois[i0 + b];
      kp.k[b] = ksk[i0 + b];
    }
    const WHoist H{digits, inputs, i0 % inputs};
    u64* t4 = (u64*)ws;
    u64* accp = t4 + (long long)nb * 2 * ell * n;
    {
      const int tiles = 16 * K, groups = (tiles + kXcds - 1) / kXcds;
      wf_rows_ip_h<<<dim3(groups * kXcds * nb), kT, 0, s>>>(G, kp, ell, beta, L, K, bmax, nb, accp, H, W.t);
      HCK_CHECK_LAUNCH();
    }
    launch_wconv_fused(WConvArgs{accp, 2LL * K * n, (long long)K * n, 0, t4, 2LL * ell * n, (long long)ell * n,
                                 W.moddown + ell, 0},
                       ell, dim3(128, 2, nb), W, s);
    HCK_CHECK_LAUNCH();
    {
      const int tiles = 16 * ell, groups = (tiles + kXcds - 1) / kXcds;
      wf_rows_ipq_h<<<dim3(groups * kXcds * nb), kT, 0, s>>>(G, kp, ell, beta, L, K, bmax, nb, t4, c0, in_stride,
                                                             out_b + (long long)i0 * out_stride,
                                                             out_a + (long long)i0 * out_stride, out_stride, H, W.t);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

}  // namespace hck
