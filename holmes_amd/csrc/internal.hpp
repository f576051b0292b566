// Device-resident CKKS context shared by every kernel translation unit of libholmes_ckks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <vector>

#include "modarith.hpp"

namespace hck {

struct WideState;  // wide.hpp: tables of a context with a prime >= 2^50

constexpr int kMaxPrimes = 64;  // Q + P primes
constexpr int kMaxAlpha = 8;    // limbs per key-switching digit (fused ModUp holds them in LDS)
constexpr int kMaxSpecial = 8;  // P primes (fused ModDown holds them in LDS)

// Base conversion constants from a source basis {b_s} to target primes {t}:
//   y_s = [x_s * hinv_s]_{b_s} (canonical),   out_t = sum_s y_s * hmod[s][t]  mod t.
// When x_s comes out of an inverse NTT, the multiplication by hinv_s rides on the transform's
// last stage: inv_n0[s] = N^-1 hinv_s and inv_n1[s] = N^-1 psi_rev_inv[1] hinv_s (mod b_s).
struct ConvConsts {
  int ns, nt;
  int src_prime[kMaxAlpha];  // prime indices of the source limbs
  int dst_prime[kMaxPrimes]; // prime index of target t
  int dst_slot[kMaxPrimes];  // position of target t in the destination buffer (limb index)
  TwPair hinv[kMaxAlpha];
  TwPair inv_n0[kMaxAlpha];
  TwPair inv_n1[kMaxAlpha];
  TwPair hmod[kMaxAlpha][kMaxPrimes];
  // Byte offset of this conversion's matrix-core table in DevTables::conv_dig (-1: none):
  // [t][c][s][a] = balanced base-256 digit c of (hmod[s][t] * 256^a mod t), centered, for
  // s < 8, a < 8 (zero for s >= ns and for a = 7), c < kConvDigits.
  long long dig_off;
  // ModDown fused with the rescale (d_mdrs): the sources are the P primes, the stored targets
  // q_0 .. q_{ell-2} with hmod[s][t] = (P / p_s mod q_t) P^-1, and q_{ell-1} rides along as
  // target nt (hmod[s][nt], dst_prime[nt]); the extra source limb Z (the q_{ell-1} limb of
  // P * d + IP) leaves its inverse transform multiplied by P^-1 through z_n0 / z_n1.
  TwPair z_n0, z_n1;
};
constexpr int kConvDigits = 7;  // balanced base-256 digits of a centered residue (|x| < 2^49)

// Per-level ModDown / rescale constants.
struct LevelConsts {
  TwPair p_inv[kMaxPrimes];     // P^-1 mod q_i (i < ell)
  TwPair qlast_inv[kMaxPrimes]; // q_{ell-1}^-1 mod q_i (i < ell - 1)
};

struct DevTables {
  int L, K, alpha, np;
  const double* p;      // [np]
  const double* pinv;   // [np]
  const double* tw_fwd; // [np][N]: psi^brv(k) (companion recomputed in mulv)
  const double* tw_inv; // [np][N]: psi^-brv(k)
  const TwPair* ninv;   // [np]: N^-1
  const TwPair* ninv_w1;// [np]: N^-1 * psi_rev_inv[1] (last inverse stage folded with N^-1)
  const TwPair* zeta4;  // [np]: psi^(N/2), a primitive 4th root of unity (multiplication by X^(N/2))
  const TwPair* pmodq;  // [np]: P = prod of the special primes, mod each prime (0 for the special ones)
  const uint8_t* conv_dig;  // digit tables of the ModUp / ModDown conversions (ConvConsts::dig_off)
};

}  // namespace hck

struct hck_context {
  int log_n, L, K, alpha, np;
  int conv_engine = 1;  // ModUp / ModDown conversion sums: 1 int8 matrix cores, 0 FP64 VALU (same results)
  hck::WideState* wide = nullptr;  // set for a context with a prime >= 2^50: every kernel runs on wide.hip
  std::vector<uint64_t> primes;
  hck::DevTables dev;
  // device allocations
  void* d_block = nullptr;            // one allocation holding all tables
  hck::ConvConsts* d_modup = nullptr; // [(L + 1) * beta_max]: index ell * beta_max + digit
  hck::ConvConsts* d_moddown = nullptr; // [L + 1]
  hck::ConvConsts* d_rescale = nullptr; // [L + 1]: level ell converts limb ell - 1 to limbs 0 .. ell - 2
  hck::ConvConsts* d_raise = nullptr;   // [L + 1]: target count t converts limb 0 to limbs 1 .. t - 1
  hck::ConvConsts* d_mdrs = nullptr;    // [L + 1]: ModDown fused with the rescale from ell to ell - 1 limbs
  hck::LevelConsts* d_level = nullptr;  // [L + 1]
  const uint64_t* d_primes_u64 = nullptr; // [np]
  const double* d_enc_twr = nullptr;      // [N/2]: special-IFFT roots, stage h at [h-1, 2h-1)
  const double* d_enc_twi = nullptr;
  std::vector<hck::ConvConsts> h_modup, h_moddown, h_rescale, h_raise, h_mdrs;
  std::vector<hck::LevelConsts> h_level;
  int beta_max;
};

namespace hck {

// A list of limbs inside one polynomial group: limb i sits at element offset off[i] * N from the
// group base and uses prime prime[i].  Passed by value as a kernel argument.
constexpr int kMaxList = 192;
struct LimbList {
  int n;
  uint16_t off[kMaxList];
  uint8_t prime[kMaxList];
};

enum Fmt { kU64 = 0, kF64 = 1 };  // canonical uint64 residues, or signed-lazy exact doubles

// Two-pass NTT launchers shared by every translation unit (ntt.hip).  Group g of `groups` starts at
// src + g * src_stride (elements); dst likewise.  Passing src == dst transforms in place.
int launch_ntt_fwd(const hck_context* c, const void* src, Fmt in, void* dst, Fmt out, int groups,
                   long long src_stride, long long dst_stride, const LimbList& list, hipStream_t s);
int launch_ntt_inv(const hck_context* c, const void* src, Fmt in, void* dst, Fmt out, int groups,
                   long long src_stride, long long dst_stride, const LimbList& list, hipStream_t s);
// Encode's rounding fused with the forward NTT: vre / vim are the special IFFT's [rows][N/2]
// outputs (natural slot order); out gets rows NTT-domain polys over `list`, overflow[row] set when a
// rounded coefficient reaches 2^61.
int launch_encode_ntt(const hck_context* c, const double* vre, const double* vim, double scale, uint64_t* out,
                      long long out_stride, int rows, int* overflow, const LimbList& list, hipStream_t s);

size_t ks_fused_bytes(const hck_context* c, int ell, int batch);
// d and add are read through sigma_galois (galois == 1: unpermuted), or through sigma of
// galois_items[b] for ciphertext b when that host array is given; acc_b / acc_a (nullable,
// unpermuted) are added to out_b / out_a, or, with ext_b / ext_a set (the key switch stops in the
// extended basis), to the extended-basis outputs.
int ks_fused(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
             const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
             const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
             char* ws, hipStream_t s, uint64_t* ext_b = nullptr, uint64_t* ext_a = nullptr,
             long long ext_stride = 0, const uint32_t* galois_items = nullptr);
// Grouped extended-basis rotations: item b = m * outputs + o (d / add at b * stride, Galois element
// galois_items[b], key ksk[b]) is member m of output o; ext[o] = acc[o] + sum_m (P sigma(add) +
// IP_b(sigma(d)), IP_a(sigma(d))).  outputs * group <= 64; workspace ks_fused_bytes(c, ell, outputs * group).
int ks_fused_sum(const hck_context* c, int ell, int outputs, int group, const uint64_t* d, long long d_stride,
                 const uint32_t* galois_items, const uint64_t* const* ksk, const uint64_t* add, long long add_stride,
                 const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride, uint64_t* ext_b,
                 uint64_t* ext_a, long long ext_stride, char* ws, hipStream_t s);
// Hoisted rotations: ks_hoist materialises the extended digits of `inputs` polys d in the full NTT
// domain ([inputs][beta][ell + K] canonical limbs, workspace ks_hoist_bytes); ks_hoisted rotates
// input i % inputs by galois[i] with ksk[i] for every item i < items from them (workspace
// ks_hoisted_bytes), bit-identical to ks_fused.  A wide context runs wide_hoist / wide_hoisted.
size_t ks_hoist_bytes(const hck_context* c, int ell, int inputs);
int ks_hoist(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride, uint64_t* digits,
             char* ws, hipStream_t s);
size_t ks_hoisted_bytes(const hck_context* c, int ell, int items);
int ks_hoisted(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
               const uint64_t* const* ksk, const uint64_t* c0, const uint64_t* c1, long long in_stride,
               const uint64_t* digits, uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws,
               hipStream_t s);
// ks_fused followed by rescale_fused in one pass: out = rescale((sigma(add) + acc_b, acc_a) +
// KeySwitch(sigma(d))) at ell - 1 limbs, bit-identical to the two steps; the q_{ell-1} limb joins
// the ModDown sources (see ConvConsts::z_n0).  add and the acc pair are nullable (relinearisation:
// acc = (d0, d1); rotation: add = c0).  Matrix-core conversion engine and ell >= 2 only: FP64
// contexts, or wide ones with wide_fused_ok (wide_ks_rescaled; HCK_ERR_UNSUPPORTED otherwise).
// Workspace ks_rs_bytes.
size_t ks_rs_bytes(const hck_context* c, int ell, int batch);
// Post-ops on the ell - 1 output limbs: out <- (twice ? 2 out : out) - sub (+ scalar[i] on out_b);
// sub_b / sub_a ([>= ell - 1] limbs per item at sub_stride) and scalar (ell - 1 canonical residues)
// nullable.  prod_ab = {a0, a1, b0, b1} (nullable): the accumulators of limbs < ell - 1 are the
// tensor terms a0 b0 and a0 b1 + a1 b0, formed in the last kernel (acc_b / acc_a then only serve
// the q_{ell-1} limb).
int ks_rescaled(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
                const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
                const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
                char* ws, hipStream_t s, int twice = 0, const uint64_t* sub_b = nullptr,
                const uint64_t* sub_a = nullptr, long long sub_stride = 0, const uint64_t* scalar = nullptr,
                const uint64_t* const* prod_ab = nullptr, long long a_stride = 0, long long b_stride = 0);
// ModDown of extended-basis polys ([ell + K] canonical limbs each) to ell limbs.
size_t moddown_bytes(const hck_context* c, int ell, int polys);
int moddown_ext(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                long long out_stride, char* ws, hipStream_t s);
// Rescale of polys from ell to ell - 1 limbs on the ModDown kernels (q_{ell-1} as the one special
// prime): out_i = (x_i - [centered x_{ell-1}]_{q_i}) * q_{ell-1}^-1.  Workspace: polys * ell limbs.
size_t rescale_bytes(const hck_context* c, int ell, int polys);
int rescale_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                  long long out_stride, char* ws, hipStream_t s);
// out[g] = rescale(sum_t w[t][.] x[g * terms + t]) from ell to ell - 1 limbs, plus the residues
// add[i] on the groups whose bit is set in add_mask (add nullable); w a device [terms][ell] table.
// groups <= 64, groups * terms <= 256.  FP64 contexts (HCK_ERR_UNSUPPORTED on a wide one).
// Workspace lincomb_rescale_bytes.
constexpr int kLcRsPtrs = 256;
constexpr int kLcRsGroups = 64;
size_t lincomb_rescale_bytes(const hck_context* c, int ell, int groups);
int lincomb_rescale(const hck_context* c, int ell, int groups, int terms, const uint64_t* const* x,
                    const uint64_t* w, uint64_t* const* out, const uint64_t* add, uint64_t add_mask, char* ws,
                    hipStream_t s);
// ModRaise of polys from one limb (q_0) to `to` limbs: the centered lift of limb 0's coefficients,
// reduced modulo q_1 .. q_{to-1} and transformed; limb 0 is copied.  Workspace: polys * to limbs.
size_t modraise_bytes(const hck_context* c, int to, int polys);
int modraise_fused(const hck_context* c, int to, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                   long long out_stride, char* ws, hipStream_t s);

// The rotation entry points' common body (keyswitch.hip): argument checks, then the fused key switch
// in launches of at most 64 items; `workspace` must hold ks_fused_bytes(ctx, level_limbs, min(batch, 64)).
int rotate_impl(const hck_context* ctx, int level_limbs, int batch, uint32_t galois, const uint32_t* galois_items,
                const uint64_t* c0, const uint64_t* c1, int64_t in_stride, const uint64_t* const* ksk,
                const uint64_t* acc0, const uint64_t* acc1, int64_t acc_stride, uint64_t* out0, uint64_t* out1,
                int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream, bool ext);

// MI355X deals consecutive workgroups to its 8 XCDs (each with its own L2) round-robin.
constexpr int kXcds = 8;

inline int beta_of(const hck_context* c, int ell) { return (ell + c->alpha - 1) / c->alpha; }
inline const ConvConsts* modup_consts(const hck_context* c, int ell, int j) {
  return c->d_modup + (size_t)ell * c->beta_max + j;
}
inline int prime_of_ext(const hck_context* c, int ell, int e) { return e < ell ? e : c->L + (e - ell); }
// Limbs per workgroup of the encoders' rounding + column kernels (grid (16, limb chunks, rows)):
// enough chunks for about 2048 workgroups.
inline int encode_limbs_per_block(int limbs, int rows) {
  int chunks = (2048 + 16 * rows - 1) / (16 * rows);
  chunks = chunks < 1 ? 1 : (chunks > limbs ? limbs : chunks);
  return (limbs + chunks - 1) / chunks;
}
// Whether two batches of n items (item i of p at p + i * p_stride, p_len words long; likewise q)
// share any word.  Strides are non-negative; a stride of 0 repeats one item.
inline bool batches_overlap(const uint64_t* p, int64_t p_stride, int64_t p_len, const uint64_t* q, int64_t q_stride,
                            int64_t q_len, int n) {
  if (n <= 0 || !p || !q) return false;
  const uint64_t* p_end = p + (int64_t)(n - 1) * p_stride + p_len;
  const uint64_t* q_end = q + (int64_t)(n - 1) * q_stride + q_len;
  return p < q_end && q < p_end;
}
}  // namespace hck

#define HCK_CHECK_LAUNCH()                         \
  do {                                             \
    hipError_t _e = hipGetLastError();             \
    if (_e != hipSuccess) return (int)_e;          \
  } while (0)
