/*
 * holmes_ckks.h -- C ABI of the MI355X-native CKKS evaluation backend (libholmes_ckks.so).
 *
 * Every entry point takes device pointers that the caller allocated (the Python host side uses
 * PyTorch-ROCm tensors) and a HIP stream passed as void*.  The library never frees caller memory.
 * Residues are uint64 in [0, q), laid out limb-major [poly][limb][N] with N = 2^16, NTT
 * (evaluation) domain unless a function says otherwise.  Return codes: 0 = success, negative =
 * argument error (HCK_ERR_*), positive = a hipError_t from the launch.
 *
 * Reference interfaces replaced (EasyFHE is not vendored in the reference; its kernel names are
 * listed in bench/cmp/report.py:26-48 and the sidecar C ABIs in bench/cmp/kernels/):
 *   hck_context_*          native context tables (`primes`, `power_of_roots(_shoup)`, `PModq`,
 *                          `QplusP_map`) read by bench/cmp/holmes_fast_stage2.py:74-82
 *   hck_ntt_forward/inverse  EasyFHE NttImpl (spec: bench/cmp/kernels/holmes_encode.cu:75-78,200-226)
 *   hck_automorphism       F.cv_hrot's NTT-domain permutation (bench/cmp/report.py:26-30)
 *   hck_keyswitch          F.cv_modup + F.cv_innerproduct_* + F.cv_moddown (report.py:26-30),
 *                          batched like giant_step_batched (bench/cmp/holmes_multi_mac.py:180-186)
 *   hck_rotate             fhe.homo_rotate (llama3fhe/operators/linear/operator.py:446-453)
 *   hck_rescale            fhe.rescale / F.cv_rescale_one_level (operator.py:387-394)
 *   hck_poly_op            F.cv_add / cv_sub / cv_neg / cv_mul / cv_mul_by_monomial (report.py:26-48)
 *   hck_poly_from_signed   the encoder's signed-integer reduction (holmes_encode.cu:108-111,133-159)
 *   hck_bsgs_mac           the multi-input BSGS baby-step MAC behind fhe.hoisted_mac_sum (its semantics are
 *                          holmes_mac.cu:8-12; per-baby pointer lists, context tables)
 *   holmes_mac_multi       holmes_mac_multi itself, with the sidecar's argument list and layouts
 *                          (holmes_mac.cu:359-402; bound at bench/cmp/holmes_multi_mac.py:49)
 *   hck_pack_diagonals     the BSGS weight diagonal packers (llama3fhe/operators/linear/weight.py:122-154,
 *                          gpu_packer.py:156-198)
 *   hck_encode             EasyFHE encode: special IFFT (cv_pre_encode_stage1) + holmes_encode_stage2
 *                          (round, reduce, NTT; holmes_encode.cu:240-285)
 *   holmes_encode_stage2   holmes_encode_stage2 itself, with the sidecar's argument list
 *                          (holmes_encode.cu:240-285; bound at bench/cmp/holmes_fast_stage2.py:37)
 *   hck_tensor / hck_relinearize / hck_mul_relin
 *                          fhe.homo_mul_no_relin / homo_relinearize / homo_mul_relin
 *                          (llama3fhe/operators/attention/prefill/qk.py:460-464,
 *                          attention/kernel_helpers.py:146-152, nonlinear/polynomial.py:140-190)
 *   hck_rotate_rescale     fhe.homo_rotate followed by fhe.rescale (operator.py:446-453, 387-394)
 *   hck_mul_relin_rescale(_postop)
 *                          fhe.homo_mul_relin_rescale_postop (nonlinear/polynomial.py:140-150): the
 *                          rescaled product, and with its double / subtract / scalar post-ops
 *   hck_weighted_sum       fhe.grouped_scalar_weighted_acc (nonlinear/polynomial.py:256-300)
 *   hck_lincomb_rescale    the evaluator's weighted sum of basis terms followed by its rescale
 *                          (nonlinear/polynomial.py:256-300)
 */
#ifndef HOLMES_CKKS_H
#define HOLMES_CKKS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HCK_OK 0
#define HCK_ERR_ARG (-1)
#define HCK_ERR_UNSUPPORTED (-2)
#define HCK_ERR_PRIME (-3)
#define HCK_ERR_ALLOC (-4)
#define HCK_ERR_WORKSPACE (-5)
#define HCK_ERR_SCRATCH (-6)

/* Bytes of the device array behind hck_rotate_noalloc (one copy per GPU, held until exit). */
#define HCK_NOALLOC_SCRATCH_BYTES (128ull << 20)

typedef struct hck_context hck_context;

/* Context over primes[0..num_q) (Q chain) followed by primes[num_q..num_q+num_p) (special
 * primes P); key-switching digits of `alpha` Q limbs.  Uploads all tables to the current device. */
int hck_context_create(hck_context** out, int log_n, int num_q, int num_p, int alpha,
                       const uint64_t* primes);
void hck_context_destroy(hck_context* ctx);
int hck_context_info(const hck_context* ctx, int* log_n, int* num_q, int* num_p, int* alpha);
/* Host copy of the root table psi^brv(k) (inverse: psi^-brv(k)) of prime `prime_idx` (N words). */
int hck_context_twiddles(const hck_context* ctx, int prime_idx, int inverse, uint64_t* out);
/* The forward root tables of every prime of the context (Q primes, then P) written to the caller's
 * device buffers, [num_q + num_p][N] uint64 each: roots[i][k] = psi_i^brv(k) and
 * roots_shoup[i][k] = floor(roots[i][k] * 2^64 / p_i).  EasyFHE's context.power_of_roots /
 * power_of_roots_shoup, the tables the encode sidecar is called with
 * (bench/cmp/holmes_fast_stage2.py:74-82).  Synchronous (set-up, not the hot path). */
int hck_context_root_tables(const hck_context* ctx, uint64_t* roots, uint64_t* roots_shoup);
const char* hck_error_string(int code);
/* Engine of the ModUp / ModDown base-conversion sums inside every key switch: 1 (default) the int8
 * matrix cores (each residue split into balanced base-256 digits, exact int32 sums), 0 FP64 VALU
 * multiply-accumulates.  Results are identical; only the timing differs.  No counterpart in the
 * reference (a scheduling knob). */
int hck_context_set_conv_engine(hck_context* ctx, int engine);

/* In-place (src == dst allowed) negacyclic NTT of `polys` x `limbs` limbs: limb l of poly b is at
 * base + b * stride + l * N and uses prime prime_idx[l] (host array).  Forward: natural-order
 * coefficients in, bit-reversed evaluation order out (out[k] = a(psi^(2 brv(k) + 1))). */
int hck_ntt_forward(const hck_context* ctx, const uint64_t* src, uint64_t* dst, int polys,
                    int64_t src_stride, int64_t dst_stride, int limbs, const int* prime_idx,
                    void* stream);
int hck_ntt_inverse(const hck_context* ctx, const uint64_t* src, uint64_t* dst, int polys,
                    int64_t src_stride, int64_t dst_stride, int limbs, const int* prime_idx,
                    void* stream);

/* sigma_g on NTT-domain limbs: out[k] = in[k'] with 2 brv(k') + 1 = g (2 brv(k) + 1) mod 2N.
 * Out-of-place only (out must not alias in). */
int hck_automorphism(const hck_context* ctx, const uint64_t* in, uint64_t* out, int polys,
                     int64_t in_stride, int64_t out_stride, int limbs, uint32_t galois,
                     void* stream);

/* Device workspace (bytes) hck_keyswitch / hck_rotate need for `batch` inputs at `level_limbs`. */
size_t hck_keyswitch_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);

/* Hybrid key switch of `batch` polynomials d[b] (level_limbs limbs, stride d_stride):
 * (out_b[b], out_a[b]) = ModDown(sum_j ModUp_j(d[b]) * ksk[b]_j) (+ add_b[b] when add_b != NULL).
 * ksk[b] (host array of device pointers) is laid out [2][beta_max][num_q + num_p][N]
 * (Q limbs, then P limbs; beta_max = ceil(num_q / alpha)).  Outputs must not alias d. */
int hck_keyswitch(const hck_context* ctx, int level_limbs, int batch, const uint64_t* d,
                  int64_t d_stride, const uint64_t* const* ksk, const uint64_t* add_b,
                  int64_t add_stride, uint64_t* out_b, uint64_t* out_a, int64_t out_stride,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Rotation of `batch` ciphertexts (c0[b], c1[b]) by galois element g with keys ksk[b]:
 * out0 = sigma(c0) + KS_b(sigma(c1)) (+ acc0[b]), out1 = KS_a(sigma(c1)) (+ acc1[b]).
 * acc0 / acc1 are both NULL or both given (the Horner giant step of a BSGS product,
 * operator.py:446-453 followed by fhe.homo_add).  Outputs may alias acc but not c0 / c1.
 * Same workspace as hck_keyswitch (hck_rotate_workspace_bytes). */
size_t hck_rotate_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);
int hck_rotate(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
               const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
               const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
               int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
               void* workspace, size_t workspace_bytes, void* stream);

/* Rotation followed by the rescale (C1's unit: INTT, automorphism, key switch, NTT, rescale):
 * outputs at level_limbs - 1 limbs (level_limbs >= 2), the residues of hck_rotate followed by
 * hck_rescale, bit for bit; fhe.homo_rotate then fhe.rescale (operator.py:446-453, 387-394).  On
 * the matrix-core conversion engine the ModDown and the rescale share one conversion pass.  The
 * outputs may not overlap c0, c1 or each other (HCK_ERR_ARG). */
size_t hck_rotate_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);
int hck_rotate_rescale(const hck_context* ctx, int level_limbs, int batch, uint32_t galois, const uint64_t* c0,
                       const uint64_t* c1, int64_t in_stride, const uint64_t* const* ksk, uint64_t* out0,
                       uint64_t* out1, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* hck_rotate without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference: it exists for those callers only.  Same arguments and results as hck_rotate; the
 * key-switch workspace is a fixed device array of HCK_NOALLOC_SCRATCH_BYTES inside the library (one
 * per GPU, resolved on the first call on that device), and nothing is allocated or freed.  The batch
 * runs in launches of as many items as the array holds at level_limbs (at most 64), one after
 * another on the stream; a level at which not even one item's key-switch workspace fits returns
 * HCK_ERR_SCRATCH without launching.  hck_rotate_noalloc_limit gives the largest batch that runs:
 * 2^30 (any batch) or 0.  Calls that overlap on one GPU (other streams or threads) race on the array;
 * calls on one stream are ordered.  Limit: a ciphertext of up to 32 limbs at K = 8, dnum 3 (24 limbs:
 * 80 MiB per item, so one item per launch). */
int hck_rotate_noalloc(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                       const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                       const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                       int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride, void* stream);
size_t hck_rotate_noalloc_limit(const hck_context* ctx, int level_limbs);

/* Rotation ending in the extended basis (hoisted form; no ModDown), fhe.fast_rotate(...,
 * output_ext=True) (llama3fhe/operators/attention/prefill/input.py:1669-1687):
 * out0 = P * sigma(c0) + IP_b(sigma(c1)) (+ acc0), out1 = IP_a(sigma(c1)) (+ acc1) over the
 * level_limbs Q primes then the K special primes (out / acc strides >= (level_limbs + K) * N words
 * per item; acc0 / acc1 both NULL or both given, and may be out0 / out1: the double-hoisted
 * giant-step sum of a BSGS product, hoist_strategy "ext_double_hoist",
 * llama3fhe/operators/linear/config.py:353-360).  hck_moddown of the pair equals hck_rotate bit
 * for bit.  Same workspace as hck_keyswitch. */
int hck_rotate_ext(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                   const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                   const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                   int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Grouped extended-basis rotations, the giant steps of a double-hoisted BSGS chunk taken `group` at
 * a time: for o < outputs,
 *   out[o] = acc[o] + sum_{m < group} (P sigma_m(c0[m][o]) + IP_b(sigma_m(c1[m][o])), IP_a(sigma_m(c1[m][o])))
 * over the level_limbs Q primes then the K special primes, item (m, o) at c0 / c1 + (m * outputs + o) *
 * in_stride, member m rotated by galois[m] with key ksk[m] (host arrays of `group`).  The running sum
 * stays on chip, so the extended accumulator is read and written once per call instead of once per
 * member (fhe.hoisted_mac_sum, "ext_double_hoist", llama3fhe/operators/linear/config.py:353-360).
 * outputs * group <= 64; out may alias acc (not c0 / c1); strides as hck_rotate_ext.  Identical
 * residues to `group` hck_rotate_ext calls accumulating in turn.  Workspace:
 * hck_rotate_workspace_bytes(ctx, level_limbs, outputs * group). */
int hck_rotate_ext_sum(const hck_context* ctx, int level_limbs, int outputs, int group, const uint32_t* galois,
                       const uint64_t* c0, const uint64_t* c1, int64_t in_stride, const uint64_t* const* ksk,
                       const uint64_t* acc0, const uint64_t* acc1, int64_t acc_stride, uint64_t* out0,
                       uint64_t* out1, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Hoisted rotations of several inputs by several amounts, the hoisted baby steps of a BSGS product
 * (fhe.prepare_hoisted_baby_rotations, llama3fhe/operators/linear/operator.py:113-119) and of a
 * bootstrap's linear transforms ("double_hoist", llama3fhe/operators/nonlinear/bootstrap.py:
 * 119-160).  hck_rotate_hoist_prepare runs the ModUp of c1 of each of `inputs` ciphertexts once and
 * stores its extended digits in the full NTT domain: `digits` (device, hck_rotate_hoist_digits_bytes
 * bytes) holds [inputs][ceil(level_limbs / alpha)][level_limbs + K] limbs.  hck_rotate_hoisted
 * then rotates input i % inputs by galois[i] with key ksk[i] for every item i < items (host arrays):
 * out[i] = (sigma(c0) + KS_b(sigma(c1)), KS_a(sigma(c1))) over level_limbs limbs, reading the
 * digits through sigma (ModUp commutes with the automorphism), so each rotation skips the INTT,
 * the conversion and the digits' NTT.  Bit-identical to hck_rotate_many.  c0 / c1 at
 * input * in_stride, out at i * out_stride.  Workspace hck_rotate_hoist_workspace_bytes(ctx,
 * level_limbs, inputs, items) serves both calls.  Both prime widths (the wide path reads the
 * digits through sigma in its inner-product kernel). */
size_t hck_rotate_hoist_digits_bytes(const hck_context* ctx, int level_limbs, int inputs);
size_t hck_rotate_hoist_workspace_bytes(const hck_context* ctx, int level_limbs, int inputs, int items);
int hck_rotate_hoist_prepare(const hck_context* ctx, int level_limbs, int inputs, const uint64_t* c1,
                             int64_t in_stride, uint64_t* digits, void* workspace, size_t workspace_bytes,
                             void* stream);
int hck_rotate_hoisted(const hck_context* ctx, int level_limbs, int inputs, int items, const uint32_t* galois,
                       const uint64_t* c0, const uint64_t* c1, int64_t in_stride, const uint64_t* digits,
                       const uint64_t* const* ksk, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                       void* workspace, size_t workspace_bytes, void* stream);

/* hck_rotate / hck_rotate_ext with a Galois element per item (galois[b], host array of `batch`):
 * one launch sequence for rotations by different amounts, each with its own key -- the batched
 * giant step of bench/cmp/holmes_multi_mac.py:180-186 (fhe.homo_rotate_batch) and the baby and
 * giant rotations of a bootstrap's linear transforms (easyfhe.bs.openfhe, "double_hoist",
 * llama3fhe/operators/nonlinear/bootstrap.py:119-160).  in_stride 0 rotates one input by every
 * element.  Same workspace as hck_keyswitch. */
int hck_rotate_many(const hck_context* ctx, int level_limbs, int batch, const uint32_t* galois,
                    const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                    const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                    int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                    void* workspace, size_t workspace_bytes, void* stream);
int hck_rotate_ext_many(const hck_context* ctx, int level_limbs, int batch, const uint32_t* galois,
                        const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                        const uint64_t* const* ksk, const uint64_t* acc0, const uint64_t* acc1,
                        int64_t acc_stride, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ModDown of `polys` extended-basis polynomials (level_limbs + K canonical NTT-domain limbs, Q
 * first) to level_limbs limbs: out = (x_Q - conv_{P->Q}(x_P)) * P^-1, fhe.moddown_from_ext
 * (input.py:1023-1029; F.cv_moddown, report.py:26-30). */
size_t hck_moddown_workspace_bytes(const hck_context* ctx, int level_limbs, int polys);
int hck_moddown(const hck_context* ctx, int level_limbs, int polys, const uint64_t* in, int64_t in_stride,
                uint64_t* out, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Rescale `polys` polynomials from level_limbs to level_limbs - 1 limbs:
 * out_i = (in_i - NTT([INTT(in_last)]_{q_i})) * q_last^-1 mod q_i. */
size_t hck_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int polys);
int hck_rescale(const hck_context* ctx, int level_limbs, int polys, const uint64_t* in,
                int64_t in_stride, uint64_t* out, int64_t out_stride, void* workspace,
                size_t workspace_bytes, void* stream);

/* ModRaise (the first step of a bootstrap, easyfhe.bs.openfhe bootstrap with
 * mode "modraise_first", llama3fhe/operators/nonlinear/bootstrap.py:119-160,626-640): `polys`
 * one-limb polynomials (limb 0 modulo q_0, NTT domain, at in + p * in_stride) lifted to to_limbs
 * limbs: out limb i = NTT_{q_i}(centered coefficients of limb 0 reduced modulo q_i). */
size_t hck_modraise_workspace_bytes(const hck_context* ctx, int to_limbs, int polys);
int hck_modraise(const hck_context* ctx, int to_limbs, int polys, const uint64_t* in, int64_t in_stride,
                 uint64_t* out, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Elementwise limb ops on [polys][limbs][N] (limb l uses prime prime_idx[l]).
 * HCK_OP_ADD/SUB/MUL: out = a op b; NEG: out = -a; MUL_SCALAR: out = a * scalar[l];
 * ADD_SCALAR: out = a + scalar[l] (a constant polynomial added in the NTT domain);
 * MUL_XHALF: out = a * X^(N/2) (NTT domain; times i on the slots); MAC: out = out + a * b. */
#define HCK_OP_ADD 0
#define HCK_OP_SUB 1
#define HCK_OP_MUL 2
#define HCK_OP_NEG 3
#define HCK_OP_MUL_SCALAR 4
#define HCK_OP_MUL_XHALF 5
#define HCK_OP_MAC 6
#define HCK_OP_ADD_SCALAR 7
int hck_poly_op(const hck_context* ctx, int op, uint64_t* out, const uint64_t* a,
                const uint64_t* b, int polys, int64_t out_stride, int64_t a_stride,
                int64_t b_stride, int limbs, const int* prime_idx, const uint64_t* scalar,
                void* stream);

/* Signed 64-bit integers (coefficient domain, N per poly) reduced to residues for each limb:
 * out[b][l][n] = in[b][n] mod q_{prime_idx[l]} in [0, q). */
int hck_poly_from_signed(const hck_context* ctx, const int64_t* in, uint64_t* out, int polys,
                         int64_t in_stride, int64_t out_stride, int limbs, const int* prime_idx,
                         void* stream);

/* BSGS baby-step MAC over `inputs` ciphertexts and `giants` giant groups:
 *   res[c][g][i][l][n] = sum_{b < babies} pts[g * babies + b][l][n] * baby_b[i][c][l][n]  (mod q_l)
 * limb l uses prime prime_idx[l] (Q limbs, or Q then P limbs for extended-basis operands).
 * baby_c0[b] / baby_c1[b] (host arrays of `babies` device pointers): components of baby rotation b,
 * [inputs][>= limbs][N] with batch stride baby_stride; pts rows [giants * babies][>= limbs][N] with
 * row stride pt_stride; res [2][giants][inputs][limbs][N] contiguous. */
int hck_bsgs_mac(const hck_context* ctx, int limbs, const int* prime_idx, int inputs, int babies, int giants,
                 const uint64_t* const* baby_c0, const uint64_t* const* baby_c1, int64_t baby_stride,
                 const uint64_t* pts, int64_t pt_stride, uint64_t* res, void* stream);

/* The reference sidecar's multi-input MAC, argument for argument (bench/cmp/kernels/holmes_mac.cu:359-402,
 * bound by ctypes at bench/cmp/holmes_multi_mac.py:49, called at :138):
 *   res[c][g][i][l][n] = sum_{b < nb} pts[g * nb + b][l][n] * baby_i[b][c][l][n]   (mod primes[l])
 * c0s / c1s: host arrays of `inputs` (1..32) device pointers to each input's baby basis
 * [nb][>= limbs][N] (baby stride bstride words); pts [groups * nb][>= limbs][N] (row stride pstride);
 * res [2][groups][inputs][limbs][N]; primes: device array, limb l modulo primes[l] (any prime below
 * 2^62).  ratios / ks (the caller's Barrett tables) are accepted and not read.  ti is the sidecar's
 * tile selector: validated against its accepted set, the tiling itself is this library's.
 * Returns -1 (inputs), -2 (nb), -3 (groups: 1..16, above 8 only with ti 10116), -4 (ti) as the
 * sidecar does, HCK_ERR_ARG for null pointers, else 0 or the HIP error of the launch. */
int holmes_mac_multi(uint64_t* res, const uint64_t* const* c0s, const uint64_t* const* c1s, long long bstride,
                     int nb, int inputs, const uint64_t* pts, long long pstride, int groups, int ti, int limbs,
                     const uint64_t* primes, const uint64_t* ratios, const uint64_t* ks, void* stream);

/* Diagonal rows of one BSGS chunk from a row-major float64 weight [dimension][dimension]:
 * out[gr * baby_steps + b][s] = W[(f - (giant_base + gr) baby_steps) mod D][(f + b + lane_shift lane) mod D],
 * f = s / lanes, lane = s % lanes, s < N/2. */
int hck_pack_diagonals(const hck_context* ctx, const double* weight, int dimension, int lanes,
                       int lane_shift, int baby_steps, int giant_base, int giant_count, double* out,
                       void* stream);

/* Encode `rows` slot vectors at `scale` into NTT-domain residues out[row][l] (row stride
 * out_row_stride words, limb l modulo prime prime_idx[l]; Q then P primes gives an
 * extended-basis plaintext).  values / values_im: float64 [rows][N/2] real and imaginary parts
 * (values_im NULL: real input).  A coefficient of magnitude >= 2^61 (the reference's encoder cap
 * MAX_ENCODED_BITS) sets overflow_flags[row] (device int array, caller-zeroed). */
size_t hck_encode_workspace_bytes(const hck_context* ctx, int rows);
int hck_encode(const hck_context* ctx, const double* values, const double* values_im, int rows, double scale,
               int limbs, const int* prime_idx, uint64_t* out, int64_t out_row_stride, void* workspace,
               size_t workspace_bytes, int* overflow_flags, void* stream);

/* The reference's encode sidecar, holmes_encode_stage2, with its argument list and return
 * convention (bench/cmp/kernels/holmes_encode.cu:240-285; bound with the argtypes of
 * bench/cmp/holmes_fast_stage2.py:37 and called as at :71-85).  out[rows][limbs][N] <- the forward
 * NTT of round(in * sf) mod primes[l]: `in` holds each row's special-IFFT output as interleaved
 * doubles (slot j: Re at 2 j, Im at 2 j + 1; row stride in_stride doubles), coefficient n < N/2
 * takes Re of slot n and n >= N/2 Im of slot n - N/2, rounded half away from zero (llround).
 * primes: device [limbs] (context.QplusP_map[limbs]); roots / roots_shoup: device [>= limbs][N]
 * (context.power_of_roots(_shoup), hck_context_root_tables).  Any prime below 2^61.  diffs, ratios,
 * ks (the sidecar's Barrett tables) and limbs_per_block are accepted and not read: residues are
 * reduced exactly by primes[l].  rows_per_launch > 0 runs the rows in batches of that many; parts
 * bit 0 runs the rounding and the NTT's column pass, bit 1 its row pass (3: the encode), bit 2 is
 * ignored (one stream).  Coefficients must stay below 2^63 in magnitude (the encoder cap is 2^61);
 * larger ones encode as 0.  Returns 0, HCK_ERR_ARG, or a hipError_t; rows <= 0 or limbs <= 0 is a
 * no-op, as in the sidecar. */
int holmes_encode_stage2(void* out, const void* in, long long in_stride, int rows, double sf, int limbs,
                         const void* primes, const void* diffs, const void* ratios, const void* ks,
                         const void* roots, const void* roots_shoup, void* stream, int rows_per_launch, int parts,
                         int limbs_per_block);

/* Tensor product of `batch` ciphertext pairs at level_limbs limbs (a = (a0, a1), b = (b0, b1), item
 * strides a_stride / b_stride): d0 = a0 b0, d1 = a0 b1 + a1 b0, d2 = a1 b1 — the three-component
 * product fhe.homo_mul_no_relin returns (llama3fhe/operators/attention/prefill/qk.py:460-464). */
int hck_tensor(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0, const uint64_t* a1,
               int64_t a_stride, const uint64_t* b0, const uint64_t* b1, int64_t b_stride, uint64_t* d0,
               uint64_t* d1, uint64_t* d2, int64_t d_stride, void* stream);

/* Relinearisation of three-component ciphertexts (d0, d1, d2) with the s^2 -> s key relin_ksk
 * (layout as for hck_keyswitch): out = (d0, d1) + KeySwitch(d2), fhe.homo_relinearize
 * (llama3fhe/operators/attention/kernel_helpers.py:146-152).  out0 / out1 may be d0 / d1, not d2. */
size_t hck_relinearize_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);
int hck_relinearize(const hck_context* ctx, int level_limbs, int batch, const uint64_t* d0, const uint64_t* d1,
                    const uint64_t* d2, int64_t in_stride, const uint64_t* relin_ksk, uint64_t* out0,
                    uint64_t* out1, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Ciphertext x ciphertext product with relinearisation: hck_tensor followed by hck_relinearize
 * (the tensor components stay in the workspace), fhe.homo_mul_relin
 * (llama3fhe/operators/nonlinear/polynomial.py:140-190, before its rescale / post-ops). */
size_t hck_mul_relin_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);
int hck_mul_relin(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0, const uint64_t* a1,
                  int64_t a_stride, const uint64_t* b0, const uint64_t* b1, int64_t b_stride,
                  const uint64_t* relin_ksk, uint64_t* out0, uint64_t* out1, int64_t out_stride, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Ciphertext x ciphertext product, relinearised and rescaled: outputs at level_limbs - 1 limbs
 * (level_limbs >= 2), the residues of hck_mul_relin followed by hck_rescale, bit for bit.  The
 * multiply-relinearise-rescale core of EasyFHE's fhe.homo_mul_relin_rescale_postop
 * (llama3fhe/operators/nonlinear/polynomial.py:140-150), its post-ops left to the caller.  On the
 * matrix-core conversion engine the ModDown and the rescale share one conversion pass (the
 * q_{level-1} limb joins the P limbs as a source); otherwise it runs the two steps.  The outputs
 * must not overlap a0, a1, b0, b1 or each other (HCK_ERR_ARG): the fused engine re-reads the
 * operands after its first store. */
size_t hck_mul_relin_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int batch);
int hck_mul_relin_rescale(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                          const uint64_t* a1, int64_t a_stride, const uint64_t* b0, const uint64_t* b1,
                          int64_t b_stride, const uint64_t* relin_ksk, uint64_t* out0, uint64_t* out1,
                          int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* hck_mul_relin_rescale with the post-ops of EasyFHE's fhe.homo_mul_relin_rescale_postop
 * (llama3fhe/operators/nonlinear/polynomial.py:140-150, the Chebyshev step T_(a+b) = 2 T_a T_b -
 * T_|a-b|): out = (apply_double ? 2 : 1) * rescale(a * b) - sub (+ scalar on out0), sub0 / sub1
 * ([>= level_limbs - 1] limbs per item at sub_stride) and scalar (level_limbs - 1 canonical
 * residues, host array) nullable; outputs must not be sub, nor overlap the operands or each other
 * (HCK_ERR_ARG).  The residues of the product followed by
 * the additions, computed in the product's last kernel on the matrix-core engine. */
int hck_mul_relin_rescale_postop(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                                 const uint64_t* a1, int64_t a_stride, const uint64_t* b0, const uint64_t* b1,
                                 int64_t b_stride, const uint64_t* relin_ksk, int apply_double, const uint64_t* sub0,
                                 const uint64_t* sub1, int64_t sub_stride, const uint64_t* scalar, uint64_t* out0,
                                 uint64_t* out1, int64_t out_stride, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Grouped scalar-weighted sum over one component of n inputs (item stride in_stride, [limbs][N]
 * each): out[g] = sum_j weights[g][j][l] * in[j] (mod q_l); weights is a device array
 * [groups][n][limbs] of residues, out items at out_stride.  fhe.grouped_scalar_weighted_acc
 * (llama3fhe/operators/nonlinear/polynomial.py:256-300). */
int hck_weighted_sum(const hck_context* ctx, int limbs, int n, int groups, const uint64_t* in, int64_t in_stride,
                     const uint64_t* weights, uint64_t* out, int64_t out_stride, void* stream);

/* Linear combinations over pointer lists: out[g] = sum_t w[t] * x[g * terms + t] over the first `limbs`
 * Q primes (limb l of every operand and output at element offset l * N from its pointer), canonical.
 * `weights` is a device [terms][limbs] table of residues shared by every group, or NULL for unit
 * weights (then the inputs must be canonical).  groups <= 64, groups * terms <= 256; an output may
 * be one of its own group's inputs.  The reference's linear combinations of ciphertexts of
 * different levels (fhe.homo_mul_scalar + homo_add chains, llama3fhe/operators/nonlinear/
 * polynomial.py:256-300) and the PairFold page append (four ciphertext sums committed together,
 * llama3fhe/operators/pairfold_kv_cache.py:400-450) in one launch. */
int hck_lincomb(const hck_context* ctx, int limbs, int groups, int terms, const uint64_t* const* x,
                const uint64_t* weights, uint64_t* const* out, void* stream);

/* A linear combination followed by the rescale: out[g] = rescale(sum_t w[t] * x[g * terms + t])
 * from level_limbs to level_limbs - 1 limbs, plus the residues add[i] (level_limbs - 1 of them,
 * canonical; add may be NULL) on the groups whose bit is set in add_mask; weights a device
 * [terms][level_limbs] table.  groups <= 64, groups * terms <= 256; an output that overlaps any
 * input of any group is refused (HCK_ERR_ARG).  The residues of hck_lincomb, hck_rescale and an HCK_OP_ADD_SCALAR, without storing the
 * combination: the Paterson-Stockmeyer step "c0 + sum c_j T_j, rescaled" of the reference's
 * evaluator (llama3fhe/operators/nonlinear/polynomial.py:256-300 followed by its rescale). */
size_t hck_lincomb_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int groups);
int hck_lincomb_rescale(const hck_context* ctx, int level_limbs, int groups, int terms, const uint64_t* const* x,
                        const uint64_t* weights, uint64_t* const* out, const uint64_t* add, uint64_t add_mask,
                        void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HOLMES_CKKS_H */
