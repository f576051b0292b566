/*
 * CPU ORACLE -- test infrastructure only.
 *
 * Plain-C, integer-only (unsigned __int128) restatement of the RNS-CKKS hot path that
 * Holmes' llama3fhe operators run through EasyFHE: prime chain, negacyclic NTT/INTT,
 * automorphism, hybrid key switching (ModUp -> key inner product -> ModDown), rescale,
 * key-switching-key generation arithmetic, and the BSGS plaintext x ciphertext MAC.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this file's
 * library, and only as the checker or the timed CPU baseline.  The product (holmes_amd/)
 * never links or calls it.  It shares no code with the HIP kernels: those use FP64-FMA
 * modular arithmetic, this file uses exact 128-bit integer arithmetic, so agreement
 * between the two is evidence for both.
 *
 * Reference anchors (EasyFHE itself is not vendored in /root/reference, see header notes):
 *  - NTT round structure and root-table order: bench/cmp/kernels/holmes_encode.cu:75-78
 *    ("Round l pairs elements n and n + 2^(15 - l) with root roots[2^l + (n >> (16 - l))]"),
 *    Cooley-Tukey butterfly holmes_encode.cu:31-37, canonical [0,p) output :219-223.
 *  - Hybrid key switch pipeline (ModUp, inner product, ModDown): kernel names
 *    bench/cmp/report.py:26-30, key layout llama3fhe/parallel/prefill/keys.py:39-47,105-117
 *    (beta digits x (limbs + K) limbs x N per component).
 *  - Rotation semantics rotate(v, r)[s] = v[(s + r) mod slots]:
 *    llama3fhe/layouts/shifted_lane.py:24-37; conjugation uses galois element 2N - 1:
 *    llama3fhe/operators/linear/complex.py:63-67.
 *  - Exact-residue BSGS MAC res[g] = sum_b pt[g*B+b] * baby[b] mod q:
 *    bench/cmp/kernels/holmes_mac.cu:8-12.
 *  - Ciphertext product (tensor, then relinearisation = key switch of d2 added to (d0, d1)) and the
 *    grouped scalar-weighted sum: the call sites qk.py:460-464, kernel_helpers.py:146-152 and
 *    nonlinear/polynomial.py:140-300 under llama3fhe/operators/.
 *
 * Parity pins for every function here live in tests/test_oracle_*.py (closed forms,
 * brute-force DFT, Python big-integer CRT, round trips).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef uint64_t u64;
typedef unsigned __int128 u128;

/* ------------------------------------------------------------------ modular helpers */
static inline u64 mulmod(u64 a, u64 b, u64 q) { return (u64)((u128)a * b % q); }
static inline u64 addmod(u64 a, u64 b, u64 q) { u64 s = a + b; return s >= q ? s - q : s; }
static inline u64 submod(u64 a, u64 b, u64 q) { return a >= b ? a - b : a + q - b; }
static u64 powmod(u64 b, u64 e, u64 q) {
  u64 r = 1 % q;
  b %= q;
  while (e) {
    if (e & 1) r = mulmod(r, b, q);
    b = mulmod(b, b, q);
    e >>= 1;
  }
  return r;
}
/* inverse of a modulo prime q (Fermat) */
static u64 invmod(u64 a, u64 q) { return powmod(a % q, q - 2, q); }
/* Shoup companion floor(w * 2^64 / q) and the exact product it enables */
static inline u64 shoup_pre(u64 w, u64 q) { return (u64)(((u128)w << 64) / q); }
static inline u64 shoup_mul(u64 a, u64 w, u64 wsh, u64 q) {
  u64 hi = (u64)(((u128)a * wsh) >> 64);
  u64 r = a * w - hi * q;
  return r >= q ? r - q : r;
}

/* Deterministic Miller-Rabin for 64-bit n (bases valid for n < 2^64). */
int or_is_prime(u64 n) {
  static const u64 bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return 0;
  for (int i = 0; i < 12; ++i) {
    if (n == bases[i]) return 1;
    if (n % bases[i] == 0) return 0;
  }
  u64 d = n - 1;
  int s = 0;
  while ((d & 1) == 0) { d >>= 1; ++s; }
  for (int i = 0; i < 12; ++i) {
    u64 x = powmod(bases[i], d, n);
    if (x == 1 || x == n - 1) continue;
    int comp = 1;
    for (int r = 1; r < s; ++r) {
      x = mulmod(x, x, n);
      if (x == n - 1) { comp = 0; break; }
    }
    if (comp) return 0;
  }
  return 1;
}

/* Prime-chain rule: candidates 2^bits + 1 - k * 2N for k = 1, 2, ... (every candidate is
 * below 2^bits and congruent to 1 mod 2N), primes taken in that descending order,
 * skipping any value listed in `exclude`.  Returns the number written (== count on success). */
int or_gen_primes(int log_n, int bits, int count, const u64* exclude, int n_excl, u64* out) {
  const u64 step = (u64)2 << log_n;
  u64 c = ((u64)1 << bits) + 1 - step;
  int got = 0;
  while (got < count && c > step) {
    if (or_is_prime(c)) {
      int skip = 0;
      for (int i = 0; i < n_excl; ++i) skip |= (exclude[i] == c);
      for (int i = 0; i < got; ++i) skip |= (out[i] == c);
      if (!skip) out[got++] = c;
    }
    c -= step;
  }
  return got;
}

/* psi = g^((q-1)/2N) for the smallest quadratic non-residue g >= 2: a primitive 2N-th root. */
u64 or_find_psi(u64 q, int log_n) {
  const u64 two_n = (u64)2 << log_n;
  for (u64 g = 2;; ++g) {
    if (powmod(g, (q - 1) / 2, q) == q - 1) return powmod(g, (q - 1) / two_n, q);
  }
}

static inline u64 bitrev(u64 x, int bits) {
  u64 r = 0;
  for (int i = 0; i < bits; ++i) { r = (r << 1) | (x & 1); x >>= 1; }
  return r;
}

/* psi_rev[k] = psi^brv(k), ipsi_rev[k] = psi^-brv(k), k < N (brv over log_n bits). */
void or_make_tables(u64 q, u64 psi, int log_n, u64* psi_rev, u64* ipsi_rev) {
  const u64 n = (u64)1 << log_n;
  const u64 ipsi = invmod(psi, q);
  u64 p = 1, ip = 1;
  for (u64 i = 0; i < n; ++i) {
    const u64 r = bitrev(i, log_n);
    psi_rev[r] = p;
    ipsi_rev[r] = ip;
    p = mulmod(p, psi, q);
    ip = mulmod(ip, ipsi, q);
  }
}

/* Forward negacyclic NTT, Cooley-Tukey, natural-order input, bit-reversed evaluation
 * order out: out[k] = sum_j a_j psi^((2 brv(k) + 1) j).  Stage l (m = 2^l) pairs j and
 * j + N/(2m) inside group i = j / (N/m) with root psi_rev[m + i]
 * (holmes_encode.cu:75-78).  Canonical [0, q) in and out. */
void or_ntt_fwd(u64* a, int log_n, u64 q, const u64* psi_rev) {
  const u64 n = (u64)1 << log_n;
  u64 t = n;
  for (u64 m = 1; m < n; m <<= 1) {
    t >>= 1;
    for (u64 i = 0; i < m; ++i) {
      const u64 w = psi_rev[m + i], wsh = shoup_pre(w, q);
      const u64 j1 = 2 * i * t;
      for (u64 j = j1; j < j1 + t; ++j) {
        const u64 u = a[j], v = shoup_mul(a[j + t], w, wsh, q);
        a[j] = addmod(u, v, q);
        a[j + t] = submod(u, v, q);
      }
    }
  }
}

/* Inverse of or_ntt_fwd: Gentleman-Sande with psi^-1 powers, then multiply by N^-1. */
void or_ntt_inv(u64* a, int log_n, u64 q, const u64* ipsi_rev) {
  const u64 n = (u64)1 << log_n;
  u64 t = 1;
  for (u64 m = n; m > 1; m >>= 1) {
    const u64 h = m >> 1;
    u64 j1 = 0;
    for (u64 i = 0; i < h; ++i) {
      const u64 w = ipsi_rev[h + i], wsh = shoup_pre(w, q);
      for (u64 j = j1; j < j1 + t; ++j) {
        const u64 u = a[j], v = a[j + t];
        a[j] = addmod(u, v, q);
        a[j + t] = shoup_mul(submod(u, v, q), w, wsh, q);
      }
      j1 += 2 * t;
    }
    t <<= 1;
  }
  const u64 ninv = invmod(n % q, q), nsh = shoup_pre(ninv, q);
  for (u64 j = 0; j < n; ++j) a[j] = shoup_mul(a[j], ninv, nsh, q);
}

/* sigma_g in the coefficient domain: a(X) -> a(X^g) mod X^N + 1 (g odd). */
void or_automorph_coeff(u64* out, const u64* in, int log_n, u64 g, u64 q) {
  const u64 n = (u64)1 << log_n, mask = 2 * n - 1;
  for (u64 i = 0; i < n; ++i) {
    const u64 e = (i * g) & mask;
    if (e < n) out[e] = in[i];
    else out[e - n] = in[i] ? q - in[i] : 0;
  }
}

/* sigma_g in the NTT domain: slot k holds a(psi^(2 brv(k) + 1)), so
 * out[k] = in[k'] with 2 brv(k') + 1 = g (2 brv(k) + 1) mod 2N. */
void or_automorph_ntt(u64* out, const u64* in, int log_n, u64 g) {
  const u64 n = (u64)1 << log_n, mask = 2 * n - 1;
  for (u64 k = 0; k < n; ++k) {
    const u64 e = ((2 * bitrev(k, log_n) + 1) * g) & mask;
    out[k] = in[bitrev((e - 1) >> 1, log_n)];
  }
}

/* ------------------------------------------------------------------ context */
typedef struct {
  int log_n, L, K, alpha;
  u64 n;
  u64* primes;   /* L + K: Q primes then P primes */
  u64* psi_rev;  /* (L + K) x N */
  u64* ipsi_rev; /* (L + K) x N */
} or_ctx;

or_ctx* or_ctx_new(int log_n, int L, int K, int alpha, const u64* primes) {
  or_ctx* c = (or_ctx*)calloc(1, sizeof(or_ctx));
  c->log_n = log_n; c->L = L; c->K = K; c->alpha = alpha;
  c->n = (u64)1 << log_n;
  const int np = L + K;
  c->primes = (u64*)malloc(sizeof(u64) * np);
  memcpy(c->primes, primes, sizeof(u64) * np);
  c->psi_rev = (u64*)malloc(sizeof(u64) * np * c->n);
  c->ipsi_rev = (u64*)malloc(sizeof(u64) * np * c->n);
  for (int i = 0; i < np; ++i) {
    const u64 psi = or_find_psi(primes[i], log_n);
    or_make_tables(primes[i], psi, log_n, c->psi_rev + (size_t)i * c->n, c->ipsi_rev + (size_t)i * c->n);
  }
  return c;
}

void or_ctx_free(or_ctx* c) {
  if (!c) return;
  free(c->primes); free(c->psi_rev); free(c->ipsi_rev); free(c);
}

void or_ctx_tables(const or_ctx* c, int prime_idx, u64* psi_rev, u64* ipsi_rev) {
  memcpy(psi_rev, c->psi_rev + (size_t)prime_idx * c->n, sizeof(u64) * c->n);
  memcpy(ipsi_rev, c->ipsi_rev + (size_t)prime_idx * c->n, sizeof(u64) * c->n);
}

static inline void ntt_f(const or_ctx* c, u64* a, int pi) { or_ntt_fwd(a, c->log_n, c->primes[pi], c->psi_rev + (size_t)pi * c->n); }
static inline void ntt_i(const or_ctx* c, u64* a, int pi) { or_ntt_inv(a, c->log_n, c->primes[pi], c->ipsi_rev + (size_t)pi * c->n); }

/* Batched NTT over `limbs` polynomials whose limb l uses prime index prime_idx[l]. */
void or_ntt_fwd_limbs(const or_ctx* c, u64* data, int limbs, const int* prime_idx) {
#pragma omp parallel for schedule(dynamic)
  for (int l = 0; l < limbs; ++l) ntt_f(c, data + (size_t)l * c->n, prime_idx[l]);
}
void or_ntt_inv_limbs(const or_ctx* c, u64* data, int limbs, const int* prime_idx) {
#pragma omp parallel for schedule(dynamic)
  for (int l = 0; l < limbs; ++l) ntt_i(c, data + (size_t)l * c->n, prime_idx[l]);
}

/* Centered fast base conversion (Bajard et al.): x given by residues x_s mod b_s (s < ns,
 * coefficient domain) -> for each target t: sum_s y_s * [(B/b_s)]_t mod t with
 * y_s = [x_s * (B/b_s)^-1]_{b_s} taken in the centered range (-b_s/2, b_s/2].  The result is the
 * residue of X + u B for the centered value X of x and an integer |u| <= (ns + 1)/2; centering
 * keeps the lift's mean at zero, so the key-switching error it multiplies has no DC bias. */
static void base_conv(const u64* const* src, const u64* src_p, int ns, u64* const* dst,
                      const u64* dst_p, int nt, u64 n) {
  u64 hinv[64];
  u64 hmod[64 * 64];
  for (int s = 0; s < ns; ++s) {
    u64 h = 1;  /* (B / b_s) mod b_s */
    for (int r = 0; r < ns; ++r) if (r != s) h = mulmod(h, src_p[r] % src_p[s], src_p[s]);
    hinv[s] = invmod(h, src_p[s]);
    for (int t = 0; t < nt; ++t) {
      u64 v = 1;  /* (B / b_s) mod t */
      for (int r = 0; r < ns; ++r) if (r != s) v = mulmod(v, src_p[r] % dst_p[t], dst_p[t]);
      hmod[s * 64 + t] = v;
    }
  }
  for (u64 j = 0; j < n; ++j) {
    u64 y[64];
    for (int s = 0; s < ns; ++s) y[s] = mulmod(src[s][j], hinv[s], src_p[s]);
    for (int t = 0; t < nt; ++t) {
      u128 pos = 0, neg = 0;
      for (int s = 0; s < ns; ++s) {
        if (2 * y[s] > src_p[s]) neg += (u128)(src_p[s] - y[s]) * hmod[s * 64 + t];
        else pos += (u128)y[s] * hmod[s * 64 + t];
      }
      const u64 tp = dst_p[t];
      dst[t][j] = (u64)(((pos % tp) + tp - (neg % tp)) % tp);
    }
  }
}

/* Digit j of level ell covers Q limbs [j*alpha, min((j+1)*alpha, ell)). */
static int digit_count(const or_ctx* c, int ell) { return (ell + c->alpha - 1) / c->alpha; }

/* ModUp of digit j: d (ell limbs, NTT domain) -> ext ((ell + K) limbs, NTT domain): limbs of
 * digit j copied from d, every other Q limb and every P limb by INTT -> base conversion from
 * the digit's primes -> NTT.  Extended limb order: Q limbs 0..ell-1, then P limbs 0..K-1. */
void or_modup(const or_ctx* c, int ell, int j, const u64* d, u64* ext) {
  const u64 n = c->n;
  const int lo = j * c->alpha, hi = (lo + c->alpha < ell) ? lo + c->alpha : ell, ns = hi - lo;
  u64* coef = (u64*)malloc(sizeof(u64) * n * ns);
  memcpy(coef, d + (size_t)lo * n, sizeof(u64) * n * ns);
  for (int s = 0; s < ns; ++s) ntt_i(c, coef + (size_t)s * n, lo + s);
  const u64* src[64]; u64 src_p[64];
  for (int s = 0; s < ns; ++s) { src[s] = coef + (size_t)s * n; src_p[s] = c->primes[lo + s]; }
  u64* dst[64]; u64 dst_p[64]; int dst_pi[64]; int nt = 0;
  for (int e = 0; e < ell + c->K; ++e) {
    const int pi = e < ell ? e : c->L + (e - ell);
    if (e >= lo && e < hi) { memcpy(ext + (size_t)e * n, d + (size_t)e * n, sizeof(u64) * n); continue; }
    dst[nt] = ext + (size_t)e * n; dst_p[nt] = c->primes[pi]; dst_pi[nt] = pi; ++nt;
  }
  base_conv(src, src_p, ns, dst, dst_p, nt, n);
  for (int t = 0; t < nt; ++t) ntt_f(c, dst[t], dst_pi[t]);
  free(coef);
}

/* ModDown: x ((ell + K) limbs, NTT domain, Q part then P part) -> out (ell limbs):
 * out_i = (x_i - NTT(conv_{P -> q_i}(INTT(x_P)))) * P^-1 mod q_i. */
void or_moddown(const or_ctx* c, int ell, const u64* x, u64* out) {
  const u64 n = c->n;
  const int K = c->K;
  u64* pc = (u64*)malloc(sizeof(u64) * n * K);
  memcpy(pc, x + (size_t)ell * n, sizeof(u64) * n * K);
  for (int k = 0; k < K; ++k) ntt_i(c, pc + (size_t)k * n, c->L + k);
  const u64* src[64]; u64 src_p[64];
  for (int k = 0; k < K; ++k) { src[k] = pc + (size_t)k * n; src_p[k] = c->primes[c->L + k]; }
  u64* dst[64]; u64 dst_p[64];
  for (int i = 0; i < ell; ++i) { dst[i] = out + (size_t)i * n; dst_p[i] = c->primes[i]; }
  base_conv(src, src_p, K, dst, dst_p, ell, n);
  for (int i = 0; i < ell; ++i) {
    const u64 q = c->primes[i];
    ntt_f(c, out + (size_t)i * n, i);
    u64 pinv = 1;
    for (int k = 0; k < K; ++k) pinv = mulmod(pinv, c->primes[c->L + k] % q, q);
    pinv = invmod(pinv, q);
    const u64* xi = x + (size_t)i * n;
    u64* oi = out + (size_t)i * n;
    for (u64 t = 0; t < n; ++t) oi[t] = mulmod(submod(xi[t], oi[t], q), pinv, q);
  }
  free(pc);
}

/* Hybrid key switch of d (ell limbs, NTT domain) with key ksk laid out
 * [2 (b, a)][beta_max = ceil(L / alpha)][L + K][N] (Q limbs 0..L-1 then P limbs):
 * (out_b, out_a) = ModDown(sum_j ModUp_j(d) * (b_j, a_j)).  Outputs ell limbs each. */
void or_keyswitch(const or_ctx* c, int ell, const u64* d, const u64* ksk, u64* out_b, u64* out_a) {
  const u64 n = c->n;
  const int ext_l = ell + c->K, beta = digit_count(c, ell), beta_max = digit_count(c, c->L);
  const size_t comp_stride = (size_t)beta_max * (c->L + c->K) * n;
  u64* ext = (u64*)malloc(sizeof(u64) * n * ext_l);
  u64* acc = (u64*)calloc((size_t)2 * ext_l * n, sizeof(u64));
  for (int j = 0; j < beta; ++j) {
    or_modup(c, ell, j, d, ext);
    for (int e = 0; e < ext_l; ++e) {
      const int pi = e < ell ? e : c->L + (e - ell);
      const u64 q = c->primes[pi];
      for (int comp = 0; comp < 2; ++comp) {
        const u64* key = ksk + comp * comp_stride + ((size_t)j * (c->L + c->K) + pi) * n;
        u64* a = acc + ((size_t)comp * ext_l + e) * n;
        const u64* x = ext + (size_t)e * n;
        for (u64 t = 0; t < n; ++t) a[t] = addmod(a[t], mulmod(x[t], key[t], q), q);
      }
    }
  }
  or_moddown(c, ell, acc, out_b);
  or_moddown(c, ell, acc + (size_t)ext_l * n, out_a);
  free(ext); free(acc);
}

/* Batched key switch for the CPU baseline: `count` independent (d, ksk) pairs, OpenMP over pairs. */
void or_keyswitch_batch(const or_ctx* c, int ell, int count, const u64* d, const u64* const* ksks,
                        u64* out_b, u64* out_a) {
  const size_t s = (size_t)ell * c->n;
#pragma omp parallel for schedule(dynamic)
  for (int i = 0; i < count; ++i) or_keyswitch(c, ell, d + i * s, ksks[i], out_b + i * s, out_a + i * s);
}

/* Rotation by galois element g of (c0, c1) at ell limbs, NTT domain: sigma_g applied to both
 * components, then (sigma(c0) + KS_b(sigma(c1)), KS_a(sigma(c1))). */
void or_rotate(const or_ctx* c, int ell, u64 g, const u64* c0, const u64* c1, const u64* ksk,
               u64* out0, u64* out1) {
  const u64 n = c->n;
  u64* r0 = (u64*)malloc(sizeof(u64) * n * ell);
  u64* r1 = (u64*)malloc(sizeof(u64) * n * ell);
  for (int i = 0; i < ell; ++i) {
    or_automorph_ntt(r0 + (size_t)i * n, c0 + (size_t)i * n, c->log_n, g);
    or_automorph_ntt(r1 + (size_t)i * n, c1 + (size_t)i * n, c->log_n, g);
  }
  or_keyswitch(c, ell, r1, ksk, out0, out1);
  for (int i = 0; i < ell; ++i) {
    const u64 q = c->primes[i];
    for (u64 t = 0; t < n; ++t) out0[(size_t)i * n + t] = addmod(out0[(size_t)i * n + t], r0[(size_t)i * n + t], q);
  }
  free(r0); free(r1);
}

/* Rescale one polynomial (ell limbs, NTT domain) to ell - 1 limbs:
 * x' = (x_i - NTT([INTT(x_last)]_{q_i})) * q_last^-1 mod q_i, the last limb's coefficients taken
 * as their centered (-q_last/2, q_last/2] representatives, so x' = round(X / q_last). */
void or_rescale(const or_ctx* c, int ell, const u64* x, u64* out) {
  const u64 n = c->n;
  const u64 ql = c->primes[ell - 1];
  u64* last = (u64*)malloc(sizeof(u64) * n);
  u64* tmp = (u64*)malloc(sizeof(u64) * n);
  memcpy(last, x + (size_t)(ell - 1) * n, sizeof(u64) * n);
  ntt_i(c, last, ell - 1);
  for (int i = 0; i < ell - 1; ++i) {
    const u64 q = c->primes[i], qinv = invmod(ql % q, q);
    for (u64 t = 0; t < n; ++t)
      tmp[t] = 2 * last[t] > ql ? (q - (ql - last[t]) % q) % q : last[t] % q;
    ntt_f(c, tmp, i);
    for (u64 t = 0; t < n; ++t)
      out[(size_t)i * n + t] = mulmod(submod(x[(size_t)i * n + t], tmp[t], q), qinv, q);
  }
  free(last); free(tmp);
}

/* Key-switching key from s_from to s_to (both ternary/small, coefficient domain int64, N each).
 * a: [beta_max][L + K][N] uniform residues (NTT domain); e: [beta_max][N] small errors
 * (coefficient domain).  ksk out: [2][beta_max][L + K][N]:
 *   b_j = -a_j * s_to + e_j + P * T_j * s_from,   a_j as given,
 * with T_j = 1 mod the primes of digit j (over the full Q chain), 0 mod other Q primes, and
 * P * T_j = 0 mod every P prime. */
void or_make_ksk(const or_ctx* c, const int64_t* s_from, const int64_t* s_to, const u64* a,
                 const int64_t* e, u64* ksk) {
  const u64 n = c->n;
  const int np = c->L + c->K, beta = digit_count(c, c->L);
  const size_t comp_stride = (size_t)beta * np * n;
  u64* sf = (u64*)malloc(sizeof(u64) * n);
  u64* st = (u64*)malloc(sizeof(u64) * n);
  u64* ee = (u64*)malloc(sizeof(u64) * n);
  for (int pi = 0; pi < np; ++pi) {
    const u64 q = c->primes[pi];
    for (u64 t = 0; t < n; ++t) {
      sf[t] = s_from[t] >= 0 ? (u64)s_from[t] % q : q - ((u64)(-s_from[t]) % q);
      st[t] = s_to[t] >= 0 ? (u64)s_to[t] % q : q - ((u64)(-s_to[t]) % q);
      if (sf[t] == q) sf[t] = 0;
      if (st[t] == q) st[t] = 0;
    }
    ntt_f(c, sf, pi);
    ntt_f(c, st, pi);
    u64 pmod = 1;
    for (int k = 0; k < c->K; ++k) pmod = mulmod(pmod, c->primes[c->L + k] % q, q);
    for (int j = 0; j < beta; ++j) {
      for (u64 t = 0; t < n; ++t) {
        const int64_t v = e[(size_t)j * n + t];
        ee[t] = v >= 0 ? (u64)v % q : (q - ((u64)(-v) % q)) % q;
      }
      ntt_f(c, ee, pi);
      const int in_digit = pi < c->L && pi / c->alpha == j;
      const u64* aj = a + ((size_t)j * np + pi) * n;
      u64* bj = ksk + ((size_t)j * np + pi) * n;
      u64* akj = ksk + comp_stride + ((size_t)j * np + pi) * n;
      for (u64 t = 0; t < n; ++t) {
        u64 v = submod(ee[t], mulmod(aj[t], st[t], q), q);
        if (in_digit) v = addmod(v, mulmod(pmod, sf[t], q), q);
        bj[t] = v;
        akj[t] = aj[t];
      }
    }
  }
  free(sf); free(st); free(ee);
}

/* Exact-residue BSGS baby-step MAC (holmes_mac.cu:8-12): for giant g < G and component c,
 *   res[c][g][limb][j] = sum_{b < nb} pt[g * nb + b][limb][j] * baby[b][c][limb][j]  mod q_limb.
 * pt: [G * nb][limbs][N]; baby: [nb][2][limbs][N]; res: [2][G][limbs][N]. */
void or_bsgs_mac(const or_ctx* c, int limbs, int nb, int G, const u64* pt, const u64* baby, u64* res) {
  const u64 n = c->n;
#pragma omp parallel for collapse(2) schedule(static)
  for (int g = 0; g < G; ++g)
    for (int l = 0; l < limbs; ++l) {
      const u64 q = c->primes[l];
      for (int comp = 0; comp < 2; ++comp) {
        u64* r = res + (((size_t)comp * G + g) * limbs + l) * n;
        for (u64 j = 0; j < n; ++j) {
          u128 acc = 0;
          for (int b = 0; b < nb; ++b)
            acc += (u128)pt[(((size_t)g * nb + b) * limbs + l) * n + j] *
                   baby[(((size_t)b * 2 + comp) * limbs + l) * n + j];
          r[j] = (u64)(acc % q);
        }
      }
    }
}

/* Elementwise helpers used by the parity tests of the product's elementwise kernels. */
void or_mul_limbs(const or_ctx* c, int limbs, const u64* a, const u64* b, u64* out) {
  for (int l = 0; l < limbs; ++l)
    for (u64 j = 0; j < c->n; ++j) out[l * c->n + j] = mulmod(a[l * c->n + j], b[l * c->n + j], c->primes[l]);
}

/* Ciphertext product before relinearisation (the textbook CKKS tensor: (a0 + a1 s)(b0 + b1 s) =
 * d0 + d1 s + d2 s^2 slotwise in the NTT domain), as fhe.homo_mul_no_relin returns it
 * (llama3fhe/operators/attention/prefill/qk.py:460-464): d0 = a0 b0, d1 = a0 b1 + a1 b0, d2 = a1 b1. */
void or_tensor(const or_ctx* c, int limbs, const u64* a0, const u64* a1, const u64* b0, const u64* b1, u64* d0,
               u64* d1, u64* d2) {
  for (int l = 0; l < limbs; ++l) {
    const u64 q = c->primes[l];
    for (u64 j = 0; j < c->n; ++j) {
      const u64 k = l * c->n + j;
      d0[k] = mulmod(a0[k], b0[k], q);
      d1[k] = addmod(mulmod(a0[k], b1[k], q), mulmod(a1[k], b0[k], q), q);
      d2[k] = mulmod(a1[k], b1[k], q);
    }
  }
}

/* out[g][l] = sum_j w[g][j][l] * x[j][l] mod q_l (fhe.grouped_scalar_weighted_acc,
 * llama3fhe/operators/nonlinear/polynomial.py:256-300). */
void or_weighted_sum(const or_ctx* c, int limbs, int n, int groups, const u64* x, const u64* w, u64* out) {
  for (int g = 0; g < groups; ++g)
    for (int l = 0; l < limbs; ++l) {
      const u64 q = c->primes[l];
      for (u64 j = 0; j < c->n; ++j) {
        u128 acc = 0;
        for (int t = 0; t < n; ++t)
          acc += (u128)w[((u64)g * n + t) * limbs + l] * x[((u64)t * limbs + l) * c->n + j] % q;
        out[((u64)g * limbs + l) * c->n + j] = (u64)(acc % q);
      }
    }
}

/* ModRaise of one NTT-domain limb modulo q_0 to `to` limbs: the centered lift c in (-q_0/2, q_0/2] of
 * its coefficients, reduced modulo q_i and transformed (the first step of a CKKS bootstrap; the
 * reference drives EasyFHE's, llama3fhe/operators/nonlinear/bootstrap.py:626-640). */
void or_modraise(const or_ctx* c, int to, const u64* in, u64* out) {
  const u64 q0 = c->primes[0];
  u64* coef = (u64*)malloc(c->n * sizeof(u64));
  memcpy(coef, in, c->n * sizeof(u64));
  ntt_i(c, coef, 0);
  for (int i = 0; i < to; ++i) {
    const u64 q = c->primes[i];
    u64* o = out + (u64)i * c->n;
    for (u64 j = 0; j < c->n; ++j) {
      const u64 v = coef[j];
      o[j] = v > q0 / 2 ? (q - (q0 - v) % q) % q : v % q;  /* v - q0 when v > q0 / 2 */
    }
    ntt_f(c, o, i);
  }
  free(coef);
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ CKKS encode (stage 1 + 2)
 * Special inverse FFT of the slot vector over the rotation group (the textbook CKKS encoder; the
 * reference's encode stage 1 feeds holmes_encode.cu:108-111, whose stage 2 rounds
 * Re(w_n) * scale into coefficient n and Im(w_n) * scale into coefficient n + slots).  Every
 * floating-point operation is written out so that the GPU encoder can perform the identical IEEE
 * sequence (this file is compiled with -ffp-contract=off):
 *   for lenh = n/2, n/4, ..., 1:  for each block i and j < lenh:
 *     u = v[i+j] + v[i+j+lenh];  d = v[i+j] - v[i+j+lenh];  v[i+j] = u;  v[i+j+lenh] = d * zeta
 *     zeta = exp(2 pi i idx / M),  idx = (lenq - (5^j mod lenq)) * (M / lenq),  lenq = 8 lenh
 *   complex product (a + bi)(c + di) = (a c - b d) + (a d + b c) i
 *   then w[k] = v[brv(k)] * (1/n);  coefficient = round-half-away(w * scale).
 * n = slots = N/2 (full packing). */
#include <math.h>

/* round half away from zero (llround semantics, holmes_encode.cu:133-159), via trunc */
static double round_away(double x) {
  double r = trunc(x);
  const double d = x - r;
  if (d >= 0.5) r += 1.0;
  else if (d <= -0.5) r -= 1.0;
  return r;
}

/* cos and sin are called through volatile pointers so that no compiler fuses them into sincos(),
 * whose results differ from separate cos/sin calls in the last bit for some arguments. */
static double (*volatile or_cos)(double) = cos;
static double (*volatile or_sin)(double) = sin;

void or_encode_twiddles(int log_n, double* tw_re, double* tw_im) {
  /* concatenated per-stage tables: stage with half-width h occupies [h - 1, 2h - 1) */
  const u64 n = (u64)1 << (log_n - 1), M = (u64)4 << (log_n - 1);
  for (u64 h = 1; h < n; h <<= 1) {
    const u64 lenq = 8 * h, gap = M / lenq;
    u64 r = 1;  /* 5^j mod M, reduced mod lenq below */
    for (u64 j = 0; j < h; ++j) {
      const u64 idx = (lenq - (r % lenq)) * gap;
      const double ang = 2.0 * M_PI * (double)idx / (double)M;
      tw_re[h - 1 + j] = or_cos(ang);
      tw_im[h - 1 + j] = or_sin(ang);
      r = (r * 5) % M;
    }
  }
}

void or_special_ifft(int log_n, double* re, double* im, const double* tw_re, const double* tw_im) {
  const u64 n = (u64)1 << (log_n - 1);
  for (u64 h = n >> 1; h >= 1; h >>= 1) {
    for (u64 i = 0; i < n; i += 2 * h) {
      for (u64 j = 0; j < h; ++j) {
        const double ar = re[i + j], ai = im[i + j], br = re[i + j + h], bi = im[i + j + h];
        const double ur = ar + br, ui = ai + bi;
        const double dr = ar - br, di = ai - bi;
        const double wr = tw_re[h - 1 + j], wi = tw_im[h - 1 + j];
        re[i + j] = ur;
        im[i + j] = ui;
        re[i + j + h] = dr * wr - di * wi;
        im[i + j + h] = dr * wi + di * wr;
      }
    }
    if (h == 1) break;
  }
}

/* values: real slot vector (n doubles).  out: [limbs][N] residues (NTT domain when ntt != 0),
 * limb l modulo the oracle context's prime prime_idx[l].  Returns -1 if a rounded coefficient is
 * 2^61 or more in magnitude (the encoder cap MAX_ENCODED_BITS = 61, llama3fhe/operators/attention/prefill/
 * softmax.py:559), else 0.  Below the cap the rounded coefficient is an exact double, reduced exactly. */
int or_encode_real(const or_ctx* c, const double* values, double scale, int limbs, const int* prime_idx,
                   int ntt, u64* out) {
  const int log_n = c->log_n;
  const u64 n = c->n >> 1, N = c->n;
  double* re = (double*)malloc(sizeof(double) * n);
  double* im = (double*)calloc(n, sizeof(double));
  double* twr = (double*)malloc(sizeof(double) * n);
  double* twi = (double*)malloc(sizeof(double) * n);
  double* coef = (double*)malloc(sizeof(double) * N);
  memcpy(re, values, sizeof(double) * n);
  or_encode_twiddles(log_n, twr, twi);
  or_special_ifft(log_n, re, im, twr, twi);
  const double inv_n = 1.0 / (double)n;
  int rc = 0;
  for (u64 k = 0; k < n; ++k) {
    const u64 s = bitrev(k, log_n - 1);
    const double wr = re[s] * inv_n, wi = im[s] * inv_n;
    coef[k] = round_away(wr * scale);
    coef[k + n] = round_away(wi * scale);
  }
  for (u64 k = 0; k < N; ++k) if (fabs(coef[k]) >= 2305843009213693952.0) rc = -1;
  for (int l = 0; l < limbs; ++l) {
    const u64 q = c->primes[prime_idx[l]];
    u64* o = out + (size_t)l * N;
    for (u64 k = 0; k < N; ++k) {
      const double v = coef[k];
      const u64 mag = (u64)fabs(v) % q;
      o[k] = v < 0 ? (mag ? q - mag : 0) : mag;
    }
    if (ntt) ntt_f(c, o, prime_idx[l]);
  }
  free(re); free(im); free(twr); free(twi); free(coef);
  return rc;
}

/* Stage 1 alone, as the encode sidecar receives it (bench/cmp/kernels/holmes_encode.cu:108-111):
 * out[2 k] = Re(w_k), out[2 k + 1] = Im(w_k), w_k = v[brv(k)] / n after the special IFFT of the
 * real slot vector `values` -- the same IEEE sequence as or_encode_real, so rounding out * scale
 * coefficient by coefficient gives that function's coefficients. */
void or_encode_stage1(const or_ctx* c, const double* values, double* out) {
  const int log_n = c->log_n;
  const u64 n = c->n >> 1;
  double* re = (double*)malloc(sizeof(double) * n);
  double* im = (double*)calloc(n, sizeof(double));
  double* twr = (double*)malloc(sizeof(double) * n);
  double* twi = (double*)malloc(sizeof(double) * n);
  memcpy(re, values, sizeof(double) * n);
  or_encode_twiddles(log_n, twr, twi);
  or_special_ifft(log_n, re, im, twr, twi);
  const double inv_n = 1.0 / (double)n;
  for (u64 k = 0; k < n; ++k) {
    const u64 s = bitrev(k, log_n - 1);
    out[2 * k] = re[s] * inv_n;
    out[2 * k + 1] = im[s] * inv_n;
  }
  free(re); free(im); free(twr); free(twi);
}

/* Diagonal packing of the BSGS weight rows (llama3fhe/operators/linear/weight.py:122-154):
 * row (g, b) of a chunk, g = giant_base + gr, gr < giant_count, b < baby_steps:
 *   row[s] = W[(f - g B) mod D][(f + b + lane_shift * lane) mod D],  f = s / lanes, lane = s % lanes. */
void or_pack_diagonals(const double* W, int D, int lanes, int lane_shift, int baby_steps, int giant_base,
                       int giant_count, int slots, double* out) {
  for (int gr = 0; gr < giant_count; ++gr) {
    const int g = giant_base + gr;
    for (int b = 0; b < baby_steps; ++b) {
      double* row = out + ((size_t)gr * baby_steps + b) * slots;
      for (int s = 0; s < slots; ++s) {
        const long f = s / lanes, lane = s % lanes;
        long o = (f - (long)g * baby_steps) % D;
        if (o < 0) o += D;
        const long in = (f + b + (long)lane_shift * lane) % D;
        row[s] = W[(size_t)o * D + in];
      }
    }
  }
}
