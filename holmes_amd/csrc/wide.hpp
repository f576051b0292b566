// The wide-prime path: contexts whose primes reach 2^50 (up to 2^61), such as the reference's
// production chain (assets/feature_major.json: 38 Q limbs of 59/60 bits, dnum 5).  The FP64 arithmetic of
// modarith.hpp is exact only below 2^50, so these contexts run every kernel on 64-bit integer words
// (modarith64.hpp: Shoup products for constants, Barrett for products of two variables) and keep
// residues canonical in [0, p) between stages.  One implementation per width: a context is either
// FP64 (every prime below 2^50) or wide, and the library's internal entry points (NTT, key switch,
// ModDown, rescale, ModRaise, encode, elementwise, tensor, MAC) dispatch on hck_context::wide.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "internal.hpp"

namespace hck {

constexpr uint64_t kWidePrimeLimit = 1ULL << 61;  // lazy sums below 4p stay inside 64 bits
constexpr int kWideChunk = 8;                      // items per key-switch launch sequence

// Fast base conversion constants (sources b_s -> targets t) with Shoup companions.
struct WideConv {
  int ns, nt;
  int src_prime[kMaxAlpha];
  int dst_prime[kMaxPrimes];
  int dst_slot[kMaxPrimes];
  uint64_t hinv[kMaxAlpha], hinv_s[kMaxAlpha];        // (B / b_s)^-1 mod b_s
  uint64_t hmod[kMaxAlpha][kMaxPrimes];               // (B / b_s) mod t
  uint64_t hmod_s[kMaxAlpha][kMaxPrimes];
  uint64_t hmod_m[kMaxAlpha][kMaxPrimes];             // (B / b_s) 2^64 mod t (Montgomery form)
  uint64_t tneg_inv[kMaxPrimes];                      // -t^-1 mod 2^64
  // The fused key switch (wide_fused.hip) runs the sources' inverse column pass in the same kernel and
  // folds hinv into its last stage: inv_n0 = N^-1 hinv, inv_n1 = N^-1 psi_rev_inv[1] hinv (mod b_s).
  uint64_t inv_n0[kMaxAlpha], inv_n0_s[kMaxAlpha], inv_n1[kMaxAlpha], inv_n1_s[kMaxAlpha];
  // The matrix-core form (wk_mconv): fold_inv[t] = fl(1 / t), the fold's quotient estimate, and the
  // offset (in 16-byte operand units) of this conversion's digit table in WideState::conv_dig.
  double fold_inv[kMaxPrimes];
  long long dig_off;
  // ModDown fused with the rescale (WideState::mdrs): sources the P primes, stored targets
  // q_0 .. q_{ell-2} with hmod[s][t] = (P / p_s mod q_t) P^-1; q_{ell-1} rides along as target nt
  // (hmod[s][nt], dst_prime[nt], no digit table), and the extra source limb Z (the q_{ell-1} limb of
  // P * acc + IP) leaves its inverse transform multiplied by P^-1: z_n0 = N^-1 P^-1,
  // z_n1 = N^-1 psi_rev_inv[1] P^-1 (mod q_{ell-1}).
  uint64_t z_n0, z_n0_s, z_n1, z_n1_s;
};

struct WideTables {
  const uint64_t* p;       // [np]
  const uint64_t* mu;      // [np] Barrett factors floor(2^(2w) / p)
  const int* w;            // [np] bit lengths
  const uint64_t* fwd;     // [np][N] psi^brv(k)
  const uint64_t* fwd_s;   // Shoup companions
  const uint64_t* inv;     // [np][N] psi^-brv(k)
  const uint64_t* inv_s;
  const uint64_t* ninv;    // [np] N^-1
  const uint64_t* ninv_s;
  const uint64_t* zeta4;   // [np] psi^(N/2)
  const uint64_t* zeta4_s;
  const uint64_t* pmod;    // [np] P mod q_i (0 for the special primes)
  const uint64_t* pmod_s;
  const uint64_t* pinv;    // [np] P^-1 mod q_i (Q primes)
  const uint64_t* pinv_s;
  const uint64_t* mneg;    // [np] -p^-1 mod 2^64 (Montgomery products of the fused key switch)
  const uint64_t* r64;     // [np] 2^64 mod p, which undoes a Montgomery product's 2^-64
  const uint64_t* r64_s;
  const uint64_t* r60;     // [np] 2^60 mod p (the split MAC's top partial sum), with its companion
  const uint64_t* r60_s;
};

struct WideState {
  WideTables t{};
  void* block = nullptr;         // one allocation for every table
  WideConv* modup = nullptr;     // [(L + 1) * beta_max]
  WideConv* moddown = nullptr;   // [L + 1]: P primes -> q_0 .. q_{ell-1}
  WideConv* rescale = nullptr;   // [L + 1]: level ell lifts q_{ell-1} to q_0 .. q_{ell-2} (the fused rescale)
  WideConv* mdrs = nullptr;      // [L + 1]: level ell's ModDown fused with the rescale (ell >= 2)
  uint64_t* qlast_inv = nullptr; // [(L + 1) * L]: level ell, prime i: q_{ell-1}^-1 mod q_i
  uint64_t* qlast_inv_s = nullptr;
  // int8 operands of the matrix-core base conversion (every modup / moddown table, at dig_off), or
  // null when a prime of the context lies below 2^46 (the fold's bound); then wk_conv runs.
  const void* conv_dig = nullptr;
  // every prime below 2^60: the fused kernels' forward passes keep their words below 16p (wide_fused.hip)
  bool primes_below_2_60 = false;
};

// Context set-up and release (context.hip calls these for a context with a prime >= 2^50).
int wide_init(hck_context* c);
void wide_free(hck_context* c);
int wide_twiddles(const hck_context* c, int prime_idx, int inverse, uint64_t* out);

// The internal entry points' wide bodies (same arguments and semantics as the FP64 ones).
int wide_ntt(const hck_context* c, const uint64_t* src, uint64_t* dst, int groups, long long src_stride,
             long long dst_stride, const LimbList& list, bool inverse, hipStream_t s);
int wide_encode_ntt(const hck_context* c, const double* vre, const double* vim, double scale, uint64_t* out,
                    long long out_stride, int rows, int* overflow, const LimbList& list, hipStream_t s);
size_t wide_ks_bytes(const hck_context* c, int ell, int batch);
int wide_ks(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
            const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
            const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
            char* ws, hipStream_t s, uint64_t* ext_b, uint64_t* ext_a, long long ext_stride,
            const uint32_t* galois_items);
// The fused key switch (wide_fused.hip): five kernels with the FP64 path's schedule, on contexts whose
// conversions run on the matrix cores (wide_fused_ok); wide_ks and wide_ks_bytes dispatch to it.
bool wide_fused_ok(const hck_context* c);
size_t wide_fused_bytes(const hck_context* c, int ell, int batch);
int wide_ks_fused(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
                  const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
                  const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a,
                  long long out_stride, char* ws, hipStream_t s, uint64_t* ext_b, uint64_t* ext_a,
                  long long ext_stride, const uint32_t* galois_items);
// ks_fused_sum's wide body on the fused kernels (same arguments; outputs * group <= 64).
int wide_ks_fused_sum(const hck_context* c, int ell, int outputs, int group, const uint64_t* d, long long d_stride,
                      const uint32_t* galois_items, const uint64_t* const* ksk, const uint64_t* add,
                      long long add_stride, const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride,
                      uint64_t* ext_b, uint64_t* ext_a, long long ext_stride, char* ws, hipStream_t s);
// ks_rescaled's wide body (same arguments and semantics): the key switch's ModDown and the rescale by
// q_{ell-1} in one conversion, on contexts with wide_fused_ok; workspace wide_fused_rs_bytes.
size_t wide_fused_rs_bytes(const hck_context* c, int ell, int batch);
int wide_ks_rescaled(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride,
                     uint32_t galois, const uint64_t* const* ksk, const uint64_t* add, long long add_stride,
                     const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride, uint64_t* out_b,
                     uint64_t* out_a, long long out_stride, char* ws, hipStream_t s, int twice,
                     const uint64_t* sub_b, const uint64_t* sub_a, long long sub_stride, const uint64_t* scalar,
                     const uint64_t* const* prod_ab, long long a_stride, long long b_stride);
size_t wide_fused_rescale_bytes(const hck_context* c, int ell, int polys);
int wide_rescale_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride,
                       uint64_t* out, long long out_stride, char* ws, hipStream_t s);
// hck_lincomb_rescale on the fused kernels: out[g] = rescale(sum_t w[t] x[g][t]) (+ add on the groups of
// add_mask) without storing the combination; workspace wide_fused_rescale_bytes(c, ell, groups).
int wide_lincomb_rescale_fused(const hck_context* c, int ell, int groups, int terms, const uint64_t* const* x,
                               const uint64_t* w, uint64_t* const* out, const uint64_t* add, uint64_t add_mask,
                               char* ws, hipStream_t s);
size_t wide_fused_moddown_bytes(const hck_context* c, int ell, int polys);
int wide_moddown_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride,
                       uint64_t* out, long long out_stride, char* ws, hipStream_t s);
size_t wide_fused_hoist_bytes(const hck_context* c, int ell, int inputs);
int wide_hoist_fused(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride,
                     uint64_t* digits, char* ws, hipStream_t s);
size_t wide_fused_hoisted_bytes(const hck_context* c, int ell, int items);
int wide_hoisted_fused(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
                       const uint64_t* const* ksk, const uint64_t* c0, long long in_stride, const uint64_t* digits,
                       uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws, hipStream_t s);
size_t wide_hoist_bytes(const hck_context* c, int ell, int inputs);
int wide_hoist(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride, uint64_t* digits,
               char* ws, hipStream_t s);
size_t wide_hoisted_bytes(const hck_context* c, int ell, int items);
int wide_hoisted(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
                 const uint64_t* const* ksk, const uint64_t* c0, const uint64_t* c1, long long in_stride,
                 const uint64_t* digits, uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws,
                 hipStream_t s);
size_t wide_moddown_bytes(const hck_context* c, int ell, int polys);
int wide_moddown(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                 long long out_stride, char* ws, hipStream_t s);
size_t wide_rescale_bytes(const hck_context* c, int ell, int polys);
int wide_rescale(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                 long long out_stride, char* ws, hipStream_t s);
size_t wide_modraise_bytes(const hck_context* c, int to, int polys);
int wide_modraise(const hck_context* c, int to, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                  long long out_stride, char* ws, hipStream_t s);
int wide_poly_op(const hck_context* c, int op, uint64_t* out, const uint64_t* a, const uint64_t* b, int polys,
                 long long out_stride, long long a_stride, long long b_stride, int limbs, const int* prime_idx,
                 const uint64_t* scalar, hipStream_t s);
int wide_tensor(const hck_context* c, int ell, int batch, const uint64_t* a0, const uint64_t* a1, long long a_stride,
                const uint64_t* b0, const uint64_t* b1, long long b_stride, uint64_t* d0, uint64_t* d1, uint64_t* d2,
                long long d_stride, hipStream_t s);
// The tensor terms a rescaled product reads (ks_rescaled with prod_ab): d2 = a1 b1 on every limb,
// d0 = a0 b0 and d1 = a0 b1 + a1 b0 on the last limb only.
int wide_tensor_d2(const hck_context* c, int ell, int batch, const uint64_t* a0, const uint64_t* a1,
                   long long a_stride, const uint64_t* b0, const uint64_t* b1, long long b_stride, uint64_t* d0,
                   uint64_t* d1, uint64_t* d2, long long d_stride, hipStream_t s);
int wide_weighted_sum(const hck_context* c, int limbs, int n, int groups, const uint64_t* in, long long in_stride,
                      const uint64_t* w, uint64_t* out, long long out_stride, hipStream_t s);
int wide_lincomb(const hck_context* c, int limbs, int groups, int terms, const uint64_t* const* x,
                 const uint64_t* w, uint64_t* const* out, hipStream_t s);
int wide_bsgs_mac(const hck_context* c, int limbs, const int* prime_idx, int inputs, int babies, int giants,
                  const uint64_t* const* baby_c0, const uint64_t* const* baby_c1, long long baby_stride,
                  const uint64_t* pts, long long pt_stride, uint64_t* res, hipStream_t s);

// holmes_encode_stage2's body: the caller's tables (primes [limbs], roots / roots_shoup [>= limbs][N]),
// any prime below 2^61; parts bit 0 runs the rounding + column pass, bit 1 the row pass.
int encode_stage2(uint64_t* out, const double* in, long long in_stride, int rows, double sf, int limbs,
                  const uint64_t* primes, const uint64_t* roots, const uint64_t* roots_shoup, int rows_per_launch,
                  int parts, hipStream_t s);

}  // namespace hck
