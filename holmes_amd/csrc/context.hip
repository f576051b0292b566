// CKKS context: prime tables, NTT twiddles and key-switching constants, resident in HBM.
//
// Replaces the native-context tables that Holmes reads through EasyFHE
// (`primes`, `barret_ratio`, `power_of_roots(_shoup)`, `PModq`, `QplusP_map`:
// bench/cmp/holmes_fast_stage2.py:74-82, bench/cmp/holmes_fast_encode.py:70-75), re-laid out for
// the FP64 arithmetic of modarith.hpp: NTT roots as exact doubles, every other constant w with its
// companion fl(w/p).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "modarith64.hpp"
#include "wide.hpp"

using u64 = uint64_t;
using u128 = unsigned __int128;

namespace {

u64 mulmod(u64 a, u64 b, u64 q) { return (u64)((u128)a * b % q); }
u64 powmod(u64 b, u64 e, u64 q) {
  u64 r = 1;
  b %= q;
  while (e) {
    if (e & 1) r = mulmod(r, b, q);
    b = mulmod(b, b, q);
    e >>= 1;
  }
  return r;
}
u64 invmod(u64 a, u64 q) { return powmod(a, q - 2, q); }

bool probable_prime(u64 n) {
  if (n < 4) return n >= 2;
  if (n % 2 == 0) return false;
  u64 d = n - 1;
  int s = 0;
  while (!(d & 1)) { d >>= 1; ++s; }
  for (u64 a : {2ULL, 325ULL, 9375ULL, 28178ULL, 450775ULL, 9780504ULL, 1795265022ULL}) {
    u64 x = powmod(a % n, d, n);
    if (a % n == 0 || x == 1 || x == n - 1) continue;
    bool composite = true;
    for (int r = 1; r < s && composite; ++r) {
      x = mulmod(x, x, n);
      if (x == n - 1) composite = false;
    }
    if (composite) return false;
  }
  return true;
}

}  // namespace

namespace hck {
// A primitive 2N-th root of unity: g^((q-1)/2N) for the smallest quadratic non-residue g (shared by
// the FP64 and the wide tables).
u64 primitive_root_2n(u64 q, int log_n) {
  const u64 two_n = (u64)2 << log_n;
  for (u64 g = 2;; ++g)
    if (powmod(g, (q - 1) / 2, q) == q - 1) return powmod(g, (q - 1) / two_n, q);
}
}  // namespace hck

namespace {

hck::TwPair pair_of(u64 w, u64 q) { return hck::TwPair{(double)w, (double)w / (double)q}; }

u64 brv(u64 x, int bits) {
  u64 r = 0;
  for (int i = 0; i < bits; ++i) { r = (r << 1) | (x & 1); x >>= 1; }
  return r;
}

// Base-conversion constants from primes src[] to primes dst[] (hmod[s][t] = prod_{r != s} b_r mod t).
// ninv[i] = N^-1 and ninv_w1[i] = N^-1 psi_rev_inv[1] mod P[i] (the inverse NTT's last-stage factors).
void fill_conv(hck::ConvConsts& cc, const std::vector<u64>& P, const std::vector<int>& src,
               const std::vector<int>& dst, const std::vector<int>& dst_slot, const std::vector<u64>& ninv,
               const std::vector<u64>& ninv_w1) {
  std::memset(&cc, 0, sizeof(cc));
  cc.ns = (int)src.size();
  cc.nt = (int)dst.size();
  for (int s = 0; s < cc.ns; ++s) {
    const u64 bs = P[src[s]];
    u64 h = 1;
    for (int r = 0; r < cc.ns; ++r) if (r != s) h = mulmod(h, P[src[r]] % bs, bs);
    cc.src_prime[s] = src[s];
    const u64 hi = invmod(h, bs);
    cc.hinv[s] = pair_of(hi, bs);
    cc.inv_n0[s] = pair_of(mulmod(ninv[src[s]], hi, bs), bs);
    cc.inv_n1[s] = pair_of(mulmod(ninv_w1[src[s]], hi, bs), bs);
    for (int t = 0; t < cc.nt; ++t) {
      const u64 qt = P[dst[t]];
      u64 v = 1;
      for (int r = 0; r < cc.ns; ++r) if (r != s) v = mulmod(v, P[src[r]] % qt, qt);
      cc.hmod[s][t] = pair_of(v, qt);
    }
  }
  for (int t = 0; t < cc.nt; ++t) { cc.dst_prime[t] = dst[t]; cc.dst_slot[t] = dst_slot[t]; }
  cc.dig_off = -1;
}

// The matrix-core table of a conversion (layout at ConvConsts::dig_off), appended to `out`.  A
// source residue y (centered, |y| < 2^49) splits into balanced digits y = sum_a d_a 256^a, a < 7;
// then y hmod[s][t] = sum_a d_a K_{s,a,t} (mod t) with K_{s,a,t} = hmod[s][t] 256^a mod t, and
// each centered K splits the same way into digits e_c: the conversion sum becomes
// sum_c 256^c sum_{s,a} d_{s,a} e_{s,a,t,c}, exact int8 products summed in int32.
bool append_conv_digits(hck::ConvConsts& cc, const std::vector<u64>& P, std::vector<uint8_t>& out) {
  constexpr int D = hck::kConvDigits;
  cc.dig_off = (long long)out.size();
  const size_t base = out.size();
  out.resize(base + (size_t)cc.nt * D * 64, 0);
  for (int t = 0; t < cc.nt; ++t) {
    const u64 qt = P[cc.dst_prime[t]];
    for (int s = 0; s < cc.ns; ++s) {
      u64 k = (u64)cc.hmod[s][t].w;  // exact: a residue below 2^50
      for (int a = 0; a < D; ++a) {
        long long v = (long long)k - (k > qt / 2 ? (long long)qt : 0);
        for (int c = 0; c < D; ++c) {
          const int d = (int)(int8_t)(uint8_t)(v & 0xFF);  // balanced digit in [-128, 127]
          out[base + (((size_t)t * D + c) * 8 + s) * 8 + a] = (uint8_t)(int8_t)d;
          v = (v - d) / 256;
        }
        if (v != 0) return false;  // cannot happen for |K| < 2^49 (seven digits reach 2^55)
        k = mulmod(k, 256 % qt, qt);
      }
    }
  }
  return true;
}

}  // namespace

extern "C" int hck_context_create(hck_context** out, int log_n, int num_q, int num_p, int alpha,
                                  const uint64_t* primes) {
  if (!out || !primes) return HCK_ERR_ARG;
  *out = nullptr;
  if (log_n != hck::kLogN) return HCK_ERR_UNSUPPORTED;
  if (num_q < 1 || num_p < 1 || num_p > hck::kMaxSpecial || alpha < 1 || alpha > hck::kMaxAlpha)
    return HCK_ERR_ARG;
  if (num_q + num_p > hck::kMaxPrimes) return HCK_ERR_ARG;
  const int np = num_q + num_p;
  const u64 two_n = (u64)2 << log_n;
  std::vector<u64> P(primes, primes + np);
  // Every prime below 2^50: the FP64 path (modarith.hpp).  Otherwise the wide path (wide.hip), for
  // primes in (2^31, 2^61).  Both need p = 1 mod 2N.
  bool wide = false;
  for (int i = 0; i < np; ++i) wide = wide || P[i] >= (1ULL << 50);
  for (int i = 0; i < np; ++i) {
    if (P[i] >= (wide ? hck::kWidePrimeLimit : (1ULL << 50)) || (wide && P[i] <= (1ULL << 31))) return HCK_ERR_PRIME;
    if (P[i] % two_n != 1 || !probable_prime(P[i])) return HCK_ERR_PRIME;
    for (int j = 0; j < i; ++j) if (P[j] == P[i]) return HCK_ERR_PRIME;
  }
  // The FP64 rescale reduces a [0, q_last) coefficient modulo q_i with one conditional subtraction.
  if (!wide)
    for (int i = 0; i < np; ++i)
      for (int j = 0; j < np; ++j)
        if (P[i] >= 2 * P[j]) return HCK_ERR_PRIME;

  hck_context* c = new (std::nothrow) hck_context();
  if (!c) return HCK_ERR_ALLOC;
  c->log_n = log_n; c->L = num_q; c->K = num_p; c->alpha = alpha; c->np = np;
  c->primes = P;
  c->beta_max = (num_q + alpha - 1) / alpha;
  const size_t n = (size_t)1 << log_n;

  // host tables
  std::vector<double> hp(np), hpinv(np);
  std::vector<double> fwd((size_t)np * n), inv((size_t)np * n);
  std::vector<hck::TwPair> ninv(np), ninv_w1(np), zeta4(np), pmodq(np);
  std::vector<u64> ninv_u(np), ninv_w1_u(np);
  for (int i = 0; i < np; ++i) {
    const u64 q = P[i];
    hp[i] = (double)q;
    hpinv[i] = 1.0 / (double)q;
    const u64 psi = hck::primitive_root_2n(q, log_n), ipsi = invmod(psi, q);
    u64 a = 1, b = 1;
    for (size_t k = 0; k < n; ++k) {
      const size_t r = brv(k, log_n);
      fwd[(size_t)i * n + r] = (double)a;
      inv[(size_t)i * n + r] = (double)b;
      a = mulmod(a, psi, q);
      b = mulmod(b, ipsi, q);
    }
    const u64 ni = invmod(n % q, q);
    ninv[i] = pair_of(ni, q);
    // the inverse transform's last stage uses psi_rev_inv[1]; folding N^-1 into it saves a pass
    ninv_u[i] = ni;
    ninv_w1_u[i] = mulmod(ni, (u64)inv[(size_t)i * n + 1], q);
    ninv_w1[i] = pair_of(ninv_w1_u[i], q);
    zeta4[i] = pair_of(powmod(psi, n / 2, q), q);
    u64 pm = 1;
    for (int k = 0; k < num_p; ++k) pm = mulmod(pm, P[num_q + k] % q, q);
    pmodq[i] = pair_of(pm, q);
  }

  // encoder roots: stage of half-width h (1 <= h < N/2) at [h - 1, 2h - 1), entry j =
  // exp(2 pi i idx / M) with idx = (lenq - (5^j mod lenq)) * (M / lenq), lenq = 8h, M = 2N
  const size_t nslots = n / 2;
  std::vector<double> etr(nslots, 0.0), eti(nslots, 0.0);
  {
    // separate cos / sin calls (a fused sincos() differs from them in the last bit for some
    // arguments); the volatile pointers keep any compiler from fusing them
    double (*volatile vcos)(double) = std::cos;
    double (*volatile vsin)(double) = std::sin;
    const u64 M = 2 * (u64)n;
    for (u64 h = 1; h < nslots; h <<= 1) {
      const u64 lenq = 8 * h, gap = M / lenq;
      u64 r = 1;
      for (u64 j = 0; j < h; ++j) {
        const u64 idx = (lenq - (r % lenq)) * gap;
        const double ang = 2.0 * M_PI * (double)idx / (double)M;
        etr[h - 1 + j] = vcos(ang);
        eti[h - 1 + j] = vsin(ang);
        r = (r * 5) % M;
      }
    }
  }

  // key-switching constants for every level ell in [1, L] and digit j
  c->h_modup.assign((size_t)(num_q + 1) * c->beta_max, hck::ConvConsts{});
  c->h_moddown.assign((size_t)(num_q + 1), hck::ConvConsts{});
  c->h_level.assign((size_t)(num_q + 1), hck::LevelConsts{});
  c->h_rescale.assign((size_t)(num_q + 1), hck::ConvConsts{});
  c->h_raise.assign((size_t)(num_q + 1), hck::ConvConsts{});
  c->h_mdrs.assign((size_t)(num_q + 1), hck::ConvConsts{});
  for (int ell = 1; ell <= num_q; ++ell) {
    const int beta = (ell + alpha - 1) / alpha;
    for (int j = 0; j < beta; ++j) {
      const int lo = j * alpha, hi = std::min(lo + alpha, ell);
      std::vector<int> src, dst, slot;
      for (int i = lo; i < hi; ++i) src.push_back(i);
      for (int e = 0; e < ell + num_p; ++e) {
        if (e >= lo && e < hi) continue;
        dst.push_back(e < ell ? e : num_q + (e - ell));
        slot.push_back(e);
      }
      fill_conv(c->h_modup[(size_t)ell * c->beta_max + j], P, src, dst, slot, ninv_u, ninv_w1_u);
    }
    std::vector<int> src, dst, slot;
    for (int k = 0; k < num_p; ++k) src.push_back(num_q + k);
    for (int i = 0; i < ell; ++i) { dst.push_back(i); slot.push_back(i); }
    fill_conv(c->h_moddown[ell], P, src, dst, slot, ninv_u, ninv_w1_u);
    if (ell >= 2) {  // rescale: the last limb is the one source, every lower limb a target
      std::vector<int> rsrc{ell - 1}, rdst, rslot;
      for (int i = 0; i < ell - 1; ++i) { rdst.push_back(i); rslot.push_back(i); }
      fill_conv(c->h_rescale[ell], P, rsrc, rdst, rslot, ninv_u, ninv_w1_u);
      // ModRaise to ell limbs: limb 0 is the one source, limbs 1 .. ell - 1 the targets
      std::vector<int> usrc{0}, udst, uslot;
      for (int i = 1; i < ell; ++i) { udst.push_back(i); uslot.push_back(i - 1); }
      fill_conv(c->h_raise[ell], P, usrc, udst, uslot, ninv_u, ninv_w1_u);
      // ModDown fused with the rescale: the moddown sums of targets q_0 .. q_{ell-2} times P^-1,
      // q_{ell-1} as the extra target nt, and P^-1 folded into the Z limb's inverse transform
      std::vector<int> fdst(dst.begin(), dst.end() - 1), fslot(slot.begin(), slot.end() - 1);
      hck::ConvConsts& fc = c->h_mdrs[ell];
      fill_conv(fc, P, src, fdst, fslot, ninv_u, ninv_w1_u);
      auto p_inv_mod = [&](u64 q) {
        u64 pm = 1;
        for (int k = 0; k < num_p; ++k) pm = mulmod(pm, P[num_q + k] % q, q);
        return invmod(pm, q);
      };
      for (int t = 0; t <= fc.nt; ++t) {
        const int qi = t < fc.nt ? fdst[t] : ell - 1;
        const u64 q = P[qi], pinv_q = p_inv_mod(q);
        for (int s = 0; s < fc.ns; ++s) {
          u64 v = 1;
          for (int r = 0; r < fc.ns; ++r) if (r != s) v = mulmod(v, P[src[r]] % q, q);
          fc.hmod[s][t] = pair_of(mulmod(v, pinv_q, q), q);
        }
      }
      fc.dst_prime[fc.nt] = ell - 1;
      fc.dst_slot[fc.nt] = ell - 1;
      const u64 ql = P[ell - 1], pinv_l = p_inv_mod(ql);
      fc.z_n0 = pair_of(mulmod(ninv_u[ell - 1], pinv_l, ql), ql);
      fc.z_n1 = pair_of(mulmod(ninv_w1_u[ell - 1], pinv_l, ql), ql);
    }
    hck::LevelConsts& lc = c->h_level[ell];
    for (int i = 0; i < ell; ++i) {
      u64 pm = 1;
      for (int k = 0; k < num_p; ++k) pm = mulmod(pm, P[num_q + k] % P[i], P[i]);
      lc.p_inv[i] = pair_of(invmod(pm, P[i]), P[i]);
      if (i < ell - 1) lc.qlast_inv[i] = pair_of(invmod(P[ell - 1] % P[i], P[i]), P[i]);
    }
  }

  // matrix-core digit tables of every ModUp and ModDown conversion
  std::vector<uint8_t> digits;
  bool digits_ok = true;
  for (hck::ConvConsts& cc : c->h_modup)   // (a wide context converts on wide.hip)
    if (cc.nt > 0 && !wide) digits_ok = digits_ok && append_conv_digits(cc, P, digits);
  for (hck::ConvConsts& cc : c->h_moddown)
    if (cc.nt > 0 && !wide) digits_ok = digits_ok && append_conv_digits(cc, P, digits);
  for (hck::ConvConsts& cc : c->h_mdrs)
    if (cc.nt > 0 && !wide) digits_ok = digits_ok && append_conv_digits(cc, P, digits);
  if (!digits_ok) { delete c; return HCK_ERR_UNSUPPORTED; }

  // one device block: [p | pinv | fwd | inv | ninv | ninv_w1 | zeta4 | pmodq | modup | moddown | level |
  // rescale | raise | moddown-rescale | primes | encoder roots | conversion digits]
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  const size_t o_p = off; off = align(off + np * sizeof(double));
  const size_t o_pinv = off; off = align(off + np * sizeof(double));
  const size_t o_fwd = off; off = align(off + fwd.size() * sizeof(double));
  const size_t o_inv = off; off = align(off + inv.size() * sizeof(double));
  const size_t o_ninv = off; off = align(off + np * sizeof(hck::TwPair));
  const size_t o_nw1 = off; off = align(off + np * sizeof(hck::TwPair));
  const size_t o_z4 = off; off = align(off + np * sizeof(hck::TwPair));
  const size_t o_pmq = off; off = align(off + np * sizeof(hck::TwPair));
  const size_t o_mu = off; off = align(off + c->h_modup.size() * sizeof(hck::ConvConsts));
  const size_t o_md = off; off = align(off + c->h_moddown.size() * sizeof(hck::ConvConsts));
  const size_t o_lv = off; off = align(off + c->h_level.size() * sizeof(hck::LevelConsts));
  const size_t o_rs = off; off = align(off + c->h_rescale.size() * sizeof(hck::ConvConsts));
  const size_t o_ra = off; off = align(off + c->h_raise.size() * sizeof(hck::ConvConsts));
  const size_t o_mr = off; off = align(off + c->h_mdrs.size() * sizeof(hck::ConvConsts));
  const size_t o_pu = off; off = align(off + np * sizeof(u64));
  const size_t o_etr = off; off = align(off + nslots * sizeof(double));
  const size_t o_eti = off; off = align(off + nslots * sizeof(double));
  const size_t o_dig = off; off = align(off + digits.size());
  void* blk = nullptr;
  hipError_t e = hipMalloc(&blk, off);
  if (e != hipSuccess) { delete c; return (int)e; }
  char* base = (char*)blk;
  struct Up { size_t o; const void* src; size_t bytes; } ups[] = {
      {o_p, hp.data(), np * sizeof(double)},
      {o_pinv, hpinv.data(), np * sizeof(double)},
      {o_fwd, fwd.data(), fwd.size() * sizeof(double)},
      {o_inv, inv.data(), inv.size() * sizeof(double)},
      {o_ninv, ninv.data(), np * sizeof(hck::TwPair)},
      {o_nw1, ninv_w1.data(), np * sizeof(hck::TwPair)},
      {o_z4, zeta4.data(), np * sizeof(hck::TwPair)},
      {o_pmq, pmodq.data(), np * sizeof(hck::TwPair)},
      {o_mu, c->h_modup.data(), c->h_modup.size() * sizeof(hck::ConvConsts)},
      {o_md, c->h_moddown.data(), c->h_moddown.size() * sizeof(hck::ConvConsts)},
      {o_lv, c->h_level.data(), c->h_level.size() * sizeof(hck::LevelConsts)},
      {o_rs, c->h_rescale.data(), c->h_rescale.size() * sizeof(hck::ConvConsts)},
      {o_ra, c->h_raise.data(), c->h_raise.size() * sizeof(hck::ConvConsts)},
      {o_mr, c->h_mdrs.data(), c->h_mdrs.size() * sizeof(hck::ConvConsts)},
      {o_pu, P.data(), np * sizeof(u64)},
      {o_etr, etr.data(), nslots * sizeof(double)},
      {o_eti, eti.data(), nslots * sizeof(double)},
      {o_dig, digits.data(), digits.size()},
  };
  for (const Up& u : ups) {
    e = hipMemcpy(base + u.o, u.src, u.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) { (void)hipFree(blk); delete c; return (int)e; }
  }
  c->d_block = blk;
  c->dev.L = num_q; c->dev.K = num_p; c->dev.alpha = alpha; c->dev.np = np;
  c->dev.p = (const double*)(base + o_p);
  c->dev.pinv = (const double*)(base + o_pinv);
  c->dev.tw_fwd = (const double*)(base + o_fwd);
  c->dev.tw_inv = (const double*)(base + o_inv);
  c->dev.ninv = (const hck::TwPair*)(base + o_ninv);
  c->dev.ninv_w1 = (const hck::TwPair*)(base + o_nw1);
  c->dev.zeta4 = (const hck::TwPair*)(base + o_z4);
  c->dev.pmodq = (const hck::TwPair*)(base + o_pmq);
  c->dev.conv_dig = (const uint8_t*)(base + o_dig);
  c->d_modup = (hck::ConvConsts*)(base + o_mu);
  c->d_moddown = (hck::ConvConsts*)(base + o_md);
  c->d_level = (hck::LevelConsts*)(base + o_lv);
  c->d_rescale = (hck::ConvConsts*)(base + o_rs);
  c->d_raise = (hck::ConvConsts*)(base + o_ra);
  c->d_mdrs = (hck::ConvConsts*)(base + o_mr);
  c->d_primes_u64 = (const u64*)(base + o_pu);
  c->d_enc_twr = (const double*)(base + o_etr);
  c->d_enc_twi = (const double*)(base + o_eti);
  if (wide) {
    const int rc = hck::wide_init(c);
    if (rc) {
      (void)hipFree(blk);
      delete c;
      return rc;
    }
  }
  *out = c;
  return HCK_OK;
}

extern "C" void hck_context_destroy(hck_context* ctx) {
  if (!ctx) return;
  hck::wide_free(ctx);
  if (ctx->d_block) (void)hipFree(ctx->d_block);
  delete ctx;
}

extern "C" int hck_context_twiddles(const hck_context* ctx, int prime_idx, int inverse, uint64_t* out) {
  if (!ctx || !out || prime_idx < 0 || prime_idx >= ctx->np) return HCK_ERR_ARG;
  if (ctx->wide) return hck::wide_twiddles(ctx, prime_idx, inverse, out);
  const size_t n = (size_t)1 << ctx->log_n;
  std::vector<double> tmp(n);
  const double* src = (inverse ? ctx->dev.tw_inv : ctx->dev.tw_fwd) + (size_t)prime_idx * n;
  hipError_t e = hipMemcpy(tmp.data(), src, n * sizeof(double), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return (int)e;
  for (size_t k = 0; k < n; ++k) out[k] = (uint64_t)tmp[k];
  return HCK_OK;
}

extern "C" int hck_context_root_tables(const hck_context* ctx, uint64_t* roots, uint64_t* roots_shoup) {
  if (!ctx || !roots || !roots_shoup) return HCK_ERR_ARG;
  const size_t n = (size_t)1 << ctx->log_n, total = (size_t)ctx->np * n;
  std::vector<uint64_t> w(total), ws(total);
  for (int i = 0; i < ctx->np; ++i) {
    const int rc = hck_context_twiddles(ctx, i, 0, w.data() + (size_t)i * n);
    if (rc) return rc;
    const uint64_t p = ctx->primes[i];
    for (size_t k = 0; k < n; ++k) ws[(size_t)i * n + k] = hck::shoup_companion(w[(size_t)i * n + k], p);
  }
  hipError_t e = hipMemcpy(roots, w.data(), total * 8, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(roots_shoup, ws.data(), total * 8, hipMemcpyHostToDevice);
  return e == hipSuccess ? HCK_OK : (int)e;
}

extern "C" int hck_context_info(const hck_context* ctx, int* log_n, int* num_q, int* num_p, int* alpha) {
  if (!ctx) return HCK_ERR_ARG;
  if (log_n) *log_n = ctx->log_n;
  if (num_q) *num_q = ctx->L;
  if (num_p) *num_p = ctx->K;
  if (alpha) *alpha = ctx->alpha;
  return HCK_OK;
}

extern "C" int hck_context_set_conv_engine(hck_context* ctx, int engine) {
  if (!ctx || engine < 0 || engine > 1) return HCK_ERR_ARG;
  ctx->conv_engine = engine;
  return HCK_OK;
}

extern "C" const char* hck_error_string(int code) {
  switch (code) {
    case HCK_OK: return "ok";
    case HCK_ERR_ARG: return "invalid argument";
    case HCK_ERR_UNSUPPORTED: return "unsupported parameter";
    case HCK_ERR_PRIME:
      return "prime rejected (needs p = 1 mod 2N, prime, distinct; all below 2^50 and within a factor 2 of each other, "
             "or any of them at or above 2^50 and all in (2^31, 2^61))";
    case HCK_ERR_ALLOC: return "host allocation failed";
    case HCK_ERR_WORKSPACE: return "workspace too small";
    case HCK_ERR_SCRATCH:
      return "request exceeds the fixed scratch of the no-allocation entry point (HCK_NOALLOC_SCRATCH_BYTES)";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
