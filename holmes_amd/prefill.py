"""Encrypted Llama-3-8B prefill layer over 128 tokens (llama3fhe/graph/prefill.py:57 ``evaluate``;
float64 semantics of llama3fhe/approx/layer.py:592-766 ``poly_prefill_layer_numpy``, Alg2 softmax at
k = 1, no prefix, all tokens valid).

    x̂  = RMSNorm1(x)                               (gamma folded into the projections)
    Q, K, V = x̂ Wq^T, x̂ Wk^T, x̂ Wv^T; RoPE on Q, K (rotate-half pairs, positions 0..127)
    S[h][q][k] = Q_h(q) . K_g(k),  g = h // 4,  k <= q
    softmax (Alg2): m = mean_k S, y = E((S - m) / (2 sqrt(d))), R = sum_k y^2,
                    lambda = rsqrt(R / n) / sqrt(n), P = (y lambda)^2        (n = q + 1 keys)
    h  = x + (P V) Wo^T
    out = h + MLP(h)                               (the C4 block: RMSNorm2, SwiGLU, down)

Layout: everything stays feature-major (the activation layout of the linear layers; slot
8 d + t of ciphertext c holds channel d of token 8 c + t), so no transposition between the
projections and attention is needed.  Channels are complex (the rotate-half pairs (f, f + 64) of a
head as x_f + i x_(f+64)), which halves the work of the projections, makes RoPE one plaintext
product with e^(i theta), and gives the real score as Re(sum_f Qz_f conj(Kz_f)):

* projection A (complex 4096 x 4096): channel 64 h + f = Qz of query head h; channel
  2048 + 64 h + f = conj Kz of KV head h // 4 (GQA replicated), RoPE'd by e^(-i theta);
* projection V: channel 64 h + f = Vz of KV head h // 4, the upper half zero;
* for every key ciphertext c' and lane offset rho the K half is lane-rotated by rho (two
  rotations, lane masks), once moved into the lower half and once kept in the upper: lane t then
  holds key 8 c' + (t + rho) mod 8;
* the 8 (c + 1) key indices j = 8 c' + rho of query ciphertext c are split over the two halves
  (j < 4 (c + 1) at channel position j of the lower half, the rest at j - 4 (c + 1) of the upper),
  so a product of Q_c (copied into both halves) with the sum of two carriers, folded over the 64
  channels of each head (six rotations), gives the scores of two keys; they are packed into one
  dense score ciphertext per query ciphertext, whose real part is the score, by baby-step /
  giant-step rotations over the channel position (14 keys);
* Alg2 on the 16 dense score ciphertexts; invalid (non-causal) positions hold score 0, so their
  exp is the public value E(0), subtracted off; row sums fold over the 128 key positions; the 16
  row-sum ciphertexts are packed into one for the inverse square root;
* PV: each pair of probability columns is broadcast over the 64 channels and multiplied with the
  lane-rotated value carriers of its two keys; the products of a query ciphertext are summed
  before one relinearisation and the two halves added; the result is complex feature-major, the
  input layout of W_O.

``PrefillAttention`` is written against the ciphertext-operation surface of ``decode.CipherOps``
(GPU) and ``tests/slot_sim.SlotOps`` (float64 slots with the same level and scale bookkeeping), so
its dataflow is checked on the CPU too; ``PrefillLayer`` adds RMSNorm, the projections, the
refresh and the MLP block on the GPU.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np

from .decode import DecodeWeights, SlotConst, _cheb, random_weights, rope_phase

__all__ = ["PrefillSpec", "PrefillPolynomials", "PrefillAttention", "PrefillLayer", "prefill_layer_numpy",
           "reference_chain_spec",
           "attention_numpy", "qk_matrix", "v_matrix", "wo_matrix", "random_weights", "attention_rotations",
           "prefill_key_rotations", "prefill_context_spec", "prefill_mlp_spec", "prefill_bootstrap_spec",
           "setup_prefill_layer"]

LANES = 8
CTS = 16
PV_INPUT_LIMBS = 5  # PV (mask + product) -> 3, W_O -> 2, residual, then the refresh
HALF = 16384
SLOTS = 32768


@dataclass(frozen=True)
class PrefillSpec:
    hidden_dim: int = 4096
    query_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 14336
    seq_len: int = 128
    rope_theta: float = 500000.0
    eps: float = 1e-5
    rms_degree: int = 15
    rms_interval: tuple = (0.5, 2.0)
    post_rms_interval: tuple = (0.5, 8.0)  # of mean(h^2) after the attention residual
    exp_degree: int = 15
    exp_interval: tuple = (-5.0, 5.0)     # of u = (S - mean_k S) / (2 sqrt(d))
    rsqrt_degree: int = 31
    rsqrt_interval: tuple = (0.9, 128.0)  # of R / n = mean_k y^2 (>= 1 by Jensen; <= n)
    silu_degree: int = 63
    silu_interval: tuple = (-16.0, 16.0)
    # refresh input bounds |slot| <= 2^bits (a two-pass refresh leaves about 2^(bits - 25)): the
    # steady layer's input is a previous layer's output (|out| below 14.3 on the synthetic workload);
    # the residual h before the MLP block stays below 7.7 there, and the block multiplies its
    # refresh error about tenfold, so its bound is the tighter one
    input_bound_bits: int = 4
    residual_bound_bits: int = 4
    # correction passes of the steady layer's series-input refreshes: the inverse square root's
    # input z maps R / n in [0.9, 128] onto [-1, 1], so near R / n = 1 an error in z moves lambda^2
    # (hence every probability) about 64 times as much; a third pass takes that refresh's error from
    # 2^-25 to below 2^-27
    exp_refresh_iterations: int = 2
    rsqrt_refresh_iterations: int = 3
    input_refresh_iterations: int = 2
    residual_refresh_iterations: int = 2

    def validate(self) -> None:
        if (self.hidden_dim, self.query_heads, self.kv_heads, self.head_dim, self.seq_len) != (4096, 32, 8, 128, 128):
            raise ValueError("the prefill layouts are built for Llama-3-8B shapes at 128 tokens")


@dataclass
class PrefillPolynomials:
    """Chebyshev series (numpy convention, argument in [-1, 1]), or the exact functions."""

    exp: object
    rsqrt: object

    @classmethod
    def fit(cls, spec: PrefillSpec) -> "PrefillPolynomials":
        from .polynomial import chebyshev_coefficients

        return cls(exp=chebyshev_coefficients(np.exp, spec.exp_degree, spec.exp_interval),
                   rsqrt=chebyshev_coefficients(lambda r: 1.0 / np.sqrt(r), spec.rsqrt_degree, spec.rsqrt_interval))


def prefill_context_spec(seed: int = 20261206, chain: str = "50"):
    """Depth 37 (38 Q limbs), dnum 5 (8-limb digits), 8 special primes: the reference's production
    structure (assets/feature_major.json).  ``chain="50"``: on 50-bit primes, scale 2^50 (the FP64
    kernels); ``chain="reference"``: the reference's own primes, a 60-bit first modulus and 59-bit Q
    primes (dcrtBits 59, firstMod 60), scale 2^59 (the 64-bit integer kernels)."""

    from .fhe import CKKSContextSpec

    if chain == "reference":
        return CKKSContextSpec(depth=37, dnum=5, dcrt_bits=59, first_mod=60, scale_bits=59,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=seed)
    if chain != "50":
        raise ValueError(f"chain must be '50' or 'reference', got {chain!r}")
    return CKKSContextSpec(depth=37, dnum=5, dcrt_bits=50, first_mod=50, scale_bits=50,
                           secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=seed)


def reference_chain_spec() -> PrefillSpec:
    """The layer's refresh schedule on the reference's 60/59-bit chain, whose one-pass bootstrap
    reaches 2^-22 (2^-13 on 50-bit primes): the exp series' input refreshed in one pass, as the
    reference refreshes its softmax checkpoint (llama3fhe/schedule.py:38-43,
    softmax_main_bootstrap_iterations = 1); the inverse square root's input in two (one pass there
    would reach the probabilities multiplied some 64-fold); the layer input and the residual in two
    (measured: one pass at both gives 2^-15.1 against the 2^-16 bar, two give 2^-17.7)."""

    return PrefillSpec(exp_refresh_iterations=1, rsqrt_refresh_iterations=2)


def prefill_mlp_spec(spec: PrefillSpec):
    """The MLP block of the layer (SwiGLU at the spec's width and polynomials)."""

    from .mlp import MLPBlockSpec

    return MLPBlockSpec(hidden_dim=spec.hidden_dim, intermediate_width=spec.intermediate,
                        silu_degree=spec.silu_degree, silu_interval=spec.silu_interval,
                        rms_degree=spec.rms_degree, rms_interval=spec.post_rms_interval, eps=spec.eps)


def prefill_bootstrap_spec(raise_limbs: int = 0):
    """The layer's refreshes: full slots, level budget (3, 3), ModRaise to ``raise_limbs`` (0: the
    top of the chain)."""

    from .bootstrap import BootstrapSpec

    return BootstrapSpec(log_slots=15, level_budget=(3, 3), raise_limbs=int(raise_limbs))


# Limbs each refresh of the layer must leave (after the two-pass correction): the residual before
# the MLP block (its 19 levels, then at least 2 for the next layer's input refresh), the steady
# layer's input (RMSNorm1 8 + projections 1, then scores 3, mean 2 and the exp series' affine map 1
# before its own refresh, which needs 2), the exp series' input (its adjust 1, the series 5, then
# y^2 / pack / affine 3 before the inverse square root's refresh, and y down to p at 5 limbs for PV),
# and the inverse square root's input (adjust 1, series 6, spread 1, y lambda 1, p 1, PV at 5).
REFRESH_LIMBS = {"residual": 21, "input": 17, "exp": 13, "rsqrt": 15}
MLP_LEVELS = 19                  # levels FeatureMajorMLPBlock takes at prefill_mlp_spec (RMSNorm2 to down_proj)
LAYER_OUTPUT_LIMBS = REFRESH_LIMBS["residual"] - MLP_LEVELS   # the next layer's input level


def refresh_raise_limbs(q_primes) -> dict:
    """ModRaise target of each refresh of the layer: the fewest limbs that leave ``REFRESH_LIMBS``."""

    from .bootstrap import raise_for_output

    spec = prefill_bootstrap_spec()
    return {k: raise_for_output(spec, q_primes, v) for k, v in REFRESH_LIMBS.items()}


# ---------------------------------------------------------------------------- float64 semantics
def _rope_heads(x: np.ndarray, heads: int, spec: PrefillSpec) -> np.ndarray:
    """RoPE of [tokens, heads * 128] at positions 0..tokens-1 (rotate-half pairs as complex)."""

    n = x.shape[0]
    ph = np.stack([rope_phase(p, spec) for p in range(n)])          # [n, 64]
    h = x.reshape(n, heads, 128)
    z = (h[:, :, :64] + 1j * h[:, :, 64:]) * ph[:, None, :]
    return np.concatenate([z.real, z.imag], axis=2).reshape(n, -1)


def attention_numpy(xn: np.ndarray, w: DecodeWeights, spec: PrefillSpec,
                    polys: PrefillPolynomials | None = None) -> dict:
    """Attention of the normalised input ``xn`` [128, 4096] (gamma applied) with this layer's
    polynomials: the residual update (P V) Wo^T and the intermediates."""

    polys = PrefillPolynomials.fit(spec) if polys is None else polys
    n = xn.shape[0]
    q = _rope_heads(xn @ w.q_proj.T, spec.query_heads, spec)
    k = _rope_heads(xn @ w.k_proj.T, spec.kv_heads, spec)
    v = xn @ w.v_proj.T
    qh = q.reshape(n, 32, 128)
    kh = k.reshape(n, 8, 128)[:, np.arange(32) // 4, :]
    vh = v.reshape(n, 8, 128)[:, np.arange(32) // 4, :]
    scores = np.einsum("qhd,khd->hqk", qh, kh)
    valid = np.tril(np.ones((n, n), dtype=bool))
    count = valid.sum(axis=1).astype(np.float64)                    # keys of each query
    mean = np.where(valid[None], scores, 0.0).sum(axis=2) / count[None, :]
    u = (scores - mean[:, :, None]) / (2.0 * math.sqrt(spec.head_dim))
    y = np.where(valid[None], _cheb(u, polys.exp, spec.exp_interval), 0.0)
    row = np.sum(y * y, axis=2)
    lam = _cheb(row / count[None, :], polys.rsqrt, spec.rsqrt_interval) / np.sqrt(count)[None, :]
    p = (y * lam[:, :, None]) ** 2
    o = np.einsum("hqk,khd->qhd", p, vh).reshape(n, -1)
    exact = np.where(valid[None], np.exp(scores / math.sqrt(spec.head_dim)), 0.0)
    exact /= exact.sum(axis=2, keepdims=True)
    return {"delta": o @ w.o_proj.T, "q": q, "k": k, "v": v, "scores": scores, "u": u, "y": y, "row_sum": row,
            "probs": p, "attn": o, "softmax_vs_exact": float(np.max(np.abs(p - exact))),
            "in_range": {"exp": bool(np.all(np.abs(u[:, valid]) <= spec.exp_interval[1])),
                         "rsqrt": bool((row / count).min() >= spec.rsqrt_interval[0]
                                       and (row / count).max() <= spec.rsqrt_interval[1])}}


def prefill_layer_numpy(x: np.ndarray, w: DecodeWeights, spec: PrefillSpec,
                        polys: PrefillPolynomials | None = None, *, exact: bool = False,
                        functions: dict | None = None) -> dict:
    """The whole layer in float64 with the layer's polynomials (the refresh is exact here);
    ``exact`` puts the functions themselves in place of every series (RMSNorm's 1 / sqrt, exp,
    the inverse square root, SiLU): a textbook Llama-3 layer.  ``functions`` replaces any of them
    by name ("rms" for both RMSNorms, "exp", "rsqrt", "silu") with another function."""

    from .mlp import mlp_block_numpy
    from .norm import rmsnorm_coefficients, rmsnorm_numpy

    x = np.asarray(x, dtype=np.float64)
    eps = float(spec.eps)
    fn = dict(functions or {})
    if exact:
        fn.setdefault("rms", lambda m: 1.0 / np.sqrt(m + eps))
        fn.setdefault("exp", np.exp)
        fn.setdefault("rsqrt", lambda r: 1.0 / np.sqrt(r))
        fn.setdefault("silu", lambda v: v / (1.0 + np.exp(-v)))
    polys = PrefillPolynomials.fit(spec) if polys is None else polys
    polys = PrefillPolynomials(exp=fn.get("exp", polys.exp), rsqrt=fn.get("rsqrt", polys.rsqrt))
    rms = {"function": fn["rms"]} if "rms" in fn else rmsnorm_coefficients(spec.rms_degree, spec.rms_interval, eps)
    xn = rmsnorm_numpy(x, w.input_layernorm, rms)
    att = attention_numpy(xn, w, spec, polys)
    h = x + att["delta"]
    mspec = prefill_mlp_spec(spec)
    out = h + mlp_block_numpy(h, w.gate_proj, w.up_proj, w.down_proj, w.post_attention_layernorm, mspec,
                              functions={k: fn[k] for k in ("rms", "silu") if k in fn})
    ms = np.mean(h * h, axis=1)
    res = {"output": out, "h": h, "xn": xn, **att}
    res["in_range"] = {**att["in_range"], "post_rms": bool(ms.min() >= spec.post_rms_interval[0]
                                                           and ms.max() <= spec.post_rms_interval[1])}
    return res


# ---------------------------------------------------------------------------- weight blocks
def _fold_rows(w: np.ndarray, heads: int) -> np.ndarray:
    """[heads * 128, in] -> complex [heads * 64, in]: row 64 h + f = w[128 h + f] + i w[128 h + f + 64]."""

    r = w.reshape(heads, 128, -1)
    return (r[:, :64] + 1j * r[:, 64:]).reshape(heads * 64, -1)


def qk_matrix(w: DecodeWeights, gamma: np.ndarray | None = None) -> np.ndarray:
    """Projection A: rows 0..2047 the query folds, 2048..4095 the conjugated key folds replicated
    over the four query heads of each KV head; gamma (RMSNorm weight) folded into the columns."""

    q = _fold_rows(w.q_proj, 32)
    k = np.conj(_fold_rows(w.k_proj, 8)).reshape(8, 64, -1)[np.arange(32) // 4].reshape(2048, -1)
    out = np.vstack([q, k])
    return out if gamma is None else out * np.asarray(gamma, dtype=np.float64)[None, :]


def v_matrix(w: DecodeWeights, gamma: np.ndarray | None = None) -> np.ndarray:
    """Projection V: rows 64 h + f the value folds of KV head h // 4, rows 2048.. zero."""

    v = _fold_rows(w.v_proj, 8).reshape(8, 64, -1)[np.arange(32) // 4].reshape(2048, -1)
    out = np.vstack([v, np.zeros_like(v)])
    return out if gamma is None else out * np.asarray(gamma, dtype=np.float64)[None, :]


def wo_matrix(w: DecodeWeights) -> np.ndarray:
    """W_O on the complex attention output: column 64 h + f = (Wo[:, 128 h + f] - i Wo[:, 128 h + f + 64]) / 2,
    so Re-doubling (x + conj x) of the product gives o Wo^T; columns 2048.. zero."""

    wo = w.o_proj.reshape(-1, 32, 128)
    cz = (wo[:, :, :64] - 1j * wo[:, :, 64:]).reshape(-1, 2048) / 2.0
    return np.hstack([cz, np.zeros_like(cz)])


# ---------------------------------------------------------------------------- slot constants
def _slot_grid():
    s = np.arange(SLOTS)
    return s // LANES, s % LANES   # channel d, lane t


def _phases(spec: PrefillSpec) -> np.ndarray:
    """[128 positions, 64 folded features] e^(i theta_f pos)."""

    return np.stack([rope_phase(p, spec) for p in range(128)])


def rope_rows(spec: PrefillSpec) -> np.ndarray:
    """[16, slots]: the query half's RoPE, channel 64 h + f of ciphertext c, lane t (token 8 c + t)
    times e^(i theta_f pos); the key half 0 (its phases ride on the key carriers' lane masks)."""

    d, t = _slot_grid()
    ph = _phases(spec)
    return np.stack([np.where(d < 2048, ph[8 * c + t, d % 64], 0.0) for c in range(CTS)])


def key_phase_masks(spec: PrefillSpec, upper: bool = False) -> list:
    """[rho] -> ([16, slots], [16, slots]): the lane masks (of one half) of the key carrier of
    ciphertext c' and lane offset rho, times the conjugate RoPE phase of the key each slot receives
    (token 8 c' + (t + rho) mod 8, folded feature f = d mod 64)."""

    d, t = _slot_grid()
    ph = np.conj(_phases(spec))
    out = []
    for rho in range(LANES):
        lo, hi = lane_masks(rho, upper)
        tok = (t + rho) % LANES
        rows = np.stack([ph[8 * c + tok, d % 64] for c in range(CTS)])
        out.append((lo[None, :] * rows, hi[None, :] * rows))
    return out


def lane_masks(rho: int, upper: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Masks of one half (the lower by default) for the two rotations of a lane rotation by rho:
    lanes t < 8 - rho (taken from the rotation by rho) and t >= 8 - rho (from the rotation by
    rho - 8)."""

    d, t = _slot_grid()
    half = (d >= 2048) if upper else (d < 2048)
    return (half & (t < LANES - rho)).astype(np.float64), (half & (t >= LANES - rho)).astype(np.float64)


def split(c: int) -> int:
    """Keys of query ciphertext c per half of its dense score ciphertext: of its 8 (c + 1) key
    indices, j < 4 (c + 1) sit at channel position j of the lower half and the others at position
    j - 4 (c + 1) of the upper half, so one product serves a key of each half."""

    return 4 * (c + 1)


def key_slot(c: int, j: int) -> int:
    """Slot offset (head 0, lane 0) of key index j in the dense score ciphertext of query c."""

    m = split(c)
    return 8 * j if j < m else HALF + 8 * (j - m)


def _carrier(j: int) -> tuple[int, int]:
    """(key ciphertext c', lane offset rho) of key index j."""

    return j // LANES, j % LANES


def validity_rows() -> np.ndarray:
    """[16, slots]: 1 where the slot of ciphertext c holds a key index j causal for query 8 c + t."""

    d, t = _slot_grid()
    pos = d % 64
    upper = d >= 2048
    rows = np.zeros((CTS, SLOTS))
    for c in range(CTS):
        m = split(c)
        j = np.where(upper, pos + m, pos)
        cp, rho = j // LANES, j % LANES
        key_lane = (t + rho) % LANES
        rows[c] = ((pos < m) & ((cp < c) | ((cp == c) & (key_lane <= t)))).astype(np.float64)
    return rows


def count_rows(power: float) -> np.ndarray:
    """[16, slots]: n^power for the query of each slot (n = 8 c + t + 1 keys), on channel
    position 0 of every head (slots 512 h + t), 0 elsewhere."""

    d, t = _slot_grid()
    at0 = ((d < 2048) & (d % 64 == 0)).astype(np.float64)
    return np.stack([at0 * (8.0 * c + t + 1.0) ** power for c in range(CTS)])


def packed_count_row(power: float) -> np.ndarray:
    """n^power at the packed row-sum position (h, c, t) of query 8 c + t."""

    d, t = _slot_grid()
    c = d % 64
    return np.where((d < 2048) & (c < CTS), (8.0 * c + t + 1.0) ** power, 0.0)


def head_row_mask(t_offset: int = 0, both: bool = False) -> np.ndarray:
    """1 on channel position 0 of every head in the lower half (slots 512 h + t), optionally shifted
    to position ``t_offset`` (slots 512 h + 8 t_offset + t); ``both``: in the upper half too."""

    d, t = _slot_grid()
    half = np.ones(d.shape, dtype=bool) if both else (d < 2048)
    return (half & (d % 64 == t_offset)).astype(np.float64)


def attention_rotations() -> tuple[int, ...]:
    """Every slot rotation of ``PrefillAttention`` (mod slots)."""

    rots = {HALF}
    for rho in range(1, LANES):
        rots |= {HALF + rho, HALF + rho - LANES, rho, rho - LANES}     # key and value carriers
    for i in range(6):
        rots |= {LANES << i, -(LANES << i)}                            # channel folds and spreads
    for b in range(1, LANES):
        rots |= {LANES * b, -LANES * b}                                # baby steps over key positions
        rots |= {64 * b, -64 * b}                                      # giant steps
    for c in range(1, CTS):
        rots |= {LANES * c, -LANES * c}                                # row-sum packing and spread
    return tuple(sorted({r % SLOTS for r in rots} - {0}))


# ---------------------------------------------------------------------------- encrypted attention
class PrefillAttention:
    """The attention core on a ciphertext-operation surface ``ops`` (decode.CipherOps or the slot
    simulator): from the projection batch A (16 items) and the value batch V (16 items) to the
    complex attention output (16 items, feature-major, the W_O input).

    Query ciphertext c has 8 (c + 1) key indices j = 8 c' + rho (key ciphertext c' <= c, lane
    offset rho); they are split over the two halves of every working ciphertext (``split``), so the
    queries are copied into both halves and one product, one channel fold and one packing rotation
    serve two keys."""

    def __init__(self, ops, spec: PrefillSpec | None = None, polys: PrefillPolynomials | None = None, *,
                 refresh_series_inputs: bool = False, series_programs: dict | None = None):
        self.ops = ops
        self._mark = lambda name: None  # stage timing callback of the running forward
        # refresh the exp series' input (16 ciphertexts, |x| <= 1) and the inverse square root's (one
        # packed ciphertext) before evaluating them: the steady-state layer, whose attention starts
        # from a refreshed layer input rather than a fresh encryption at the top of the chain
        # (the reference's refresh_softmax_exp_inputs, llama3fhe/graph/prefill.py:134-221)
        self.refresh_series_inputs = bool(refresh_series_inputs)
        self._taps = None
        self.series_programs = dict(series_programs or {})  # "exp" / "rsqrt" -> program (default: ops')
        self.spec = PrefillSpec() if spec is None else spec
        self.spec.validate()
        self.polys = PrefillPolynomials.fit(self.spec) if polys is None else polys
        self.lane = {hf: [tuple(SlotConst(m) for m in lane_masks(rho, hf)) for rho in range(LANES)]
                     for hf in (False, True)}
        valid = validity_rows()
        self.invalid = SlotConst(1.0 - valid)
        self.row0 = SlotConst(head_row_mask(0))
        self.row0_both = SlotConst(head_row_mask(0, both=True))
        self.rope_q = SlotConst(rope_rows(self.spec))
        self.key_masks = {hf: [tuple(SlotConst(m) for m in pair) for pair in key_phase_masks(self.spec, hf)]
                          for hf in (False, True)}
        d, t = _slot_grid()
        n_rows = np.stack([8.0 * c + t + 1.0 for c in range(CTS)])
        self.valid_over_n = SlotConst(valid / n_rows)
        self.inv_sqrt_count = SlotConst(count_rows(-0.5))
        self.rowc = [SlotConst(head_row_mask(c)) for c in range(CTS)]
        self.pairs = [(c, p) for c in range(CTS) for p in range(split(c))]
        self.pair_budget = 320
        a_e, b_e = (float(v) for v in self.spec.exp_interval)
        # poly argument x = (2 u - (a + b)) / (b - a) with u = S / (2 sqrt d) and 2 Re = D + conj D = 2 S
        self.exp_alpha = 1.0 / (2.0 * math.sqrt(self.spec.head_dim)) / (b_e - a_e)
        self.exp_beta = -(a_e + b_e) / (b_e - a_e)
        self.exp_alpha_valid = SlotConst(self.exp_alpha * valid)
        self.exp_at_zero = float(_cheb(0.0, self.polys.exp, self.spec.exp_interval))
        a_r, b_r = (float(v) for v in self.spec.rsqrt_interval)
        self.rs_alpha, self.rs_beta = 2.0 / (b_r - a_r), -(a_r + b_r) / (b_r - a_r)
        self.rs_in = SlotConst(self.rs_alpha * packed_count_row(-1.0))
        self.rs_shift = SlotConst(self.rs_beta * (packed_count_row(1.0) > 0))

    # -- carriers
    def _lane_carriers(self, X, *sets):
        """For each (base, masks) of ``sets``: items (c', rho) for rho = 0..7 of the batch X, X rotated
        by ``base`` with lanes rotated by rho (lane t holds token 8 c' + (t + rho) mod 8), kept on the
        half ``masks`` [rho] selects (per-item rows allowed).  Every rotation of X comes from one
        hoisted ModUp per item (15 offsets per set)."""

        ops = self.ops
        offs = [o for base, _ in sets for o in [base] + [b for rho in range(1, LANES)
                                                          for b in (base + rho, base + rho - LANES)]]
        rot = dict(zip(offs, ops.rotate_offsets(X, offs)))
        result = []
        for base, masks in sets:
            out = []
            for rho in range(LANES):
                lo, hi = masks[rho]
                if rho == 0:
                    out.append(ops.mac([(rot[base], lo)]))
                else:
                    out.append(ops.mac([(rot[base + rho], lo), (rot[base + rho - LANES], hi)]))
            items = [ops.items(o) for o in out]             # [rho][c']
            result.append({(cp, rho): items[rho][cp] for cp in range(CTS) for rho in range(LANES)})
        return result

    def _pair_carriers(self, low, up, pairs):
        """Per pair (c, p): the carrier of key p in the lower half plus that of key p + split(c) in
        the upper half (one batch)."""

        ops = self.ops
        lo = ops.batch([low[_carrier(p)] for _, p in pairs])
        hi = ops.batch([up[_carrier(p + split(c))] for c, p in pairs])
        return ops.add(lo, hi)

    def _query_groups(self):
        """Consecutive query ciphertexts whose (c, p) products form one batch of at most
        ``pair_budget`` items (the products of all pairs at once would need tens of GB)."""

        groups, cur, n = [], [], 0
        for c in range(CTS):
            k = split(c)
            if cur and n + k > self.pair_budget:
                groups.append(cur)
                cur, n = [], 0
            cur.append(c)
            n += k
        groups.append(cur)
        return groups

    def _pack_keys(self, m, group):
        """Dense score ciphertexts of the query ciphertexts in ``group`` from the channel sums
        m[(c, p)] (masked to position 0 of both halves): sum_p rot(m_p, -8 p) with p = 8 a + b, the
        baby rotations by -8 b of the whole group in one batch, their sums over b, then the giant
        rotations by -64 a in one batch and the sums over a."""

        ops = self.ops
        pairs = [(c, p) for c in group for p in range(split(c))]
        baby = ops.items(ops.rotate(ops.batch([m[x] for x in pairs]), [-LANES * (p % LANES) for _, p in pairs]))
        baby = dict(zip(pairs, baby))
        giants = [(c, a) for c in group for a in range((split(c) + LANES - 1) // LANES)]
        acc = [baby[(c, LANES * a)] for c, a in giants]
        for b in range(1, LANES):
            sel = [i for i, (c, a) in enumerate(giants) if LANES * a + b < split(c)]
            s = ops.add(ops.batch([acc[i] for i in sel]),
                        ops.batch([baby[(giants[i][0], LANES * giants[i][1] + b)] for i in sel]))
            for i, item in zip(sel, ops.items(s)):
                acc[i] = item
        del baby
        moved = dict(zip(giants, ops.items(ops.rotate(ops.batch(acc), [-64 * a for _, a in giants]))))
        out = {c: moved[(c, 0)] for c in group}
        for a in range(1, LANES):
            cs = [c for c in group if (c, a) in moved]
            if cs:
                summed = ops.add(ops.batch([out[c] for c in cs]), ops.batch([moved[(c, a)] for c in cs]))
                out.update(zip(cs, ops.items(summed)))
        return out

    def scores(self, A):
        """Dense score ciphertexts D_c (16 items): 2 S at key index j's slot (``key_slot``), 0 where
        no key is computed; ``A`` the projection batch (before RoPE)."""

        ops = self.ops
        # the key half moved down, and kept in place
        k_lo, k_up = self._lane_carriers(A, (HALF, self.key_masks[False]), (0, self.key_masks[True]))
        q = ops.mac([(A, self.rope_q)])                               # RoPE'd queries, lower half
        q = ops.items(ops.add(q, ops.rotate(q, HALF)))                # ... in both halves
        dense = {}
        for group in self._query_groups():
            pairs = [(c, p) for c in group for p in range(split(c))]
            right = self._pair_carriers(k_lo, k_up, pairs)
            prod = ops.mul(ops.batch([q[c] for c, _ in pairs]), right)
            del right
            for i in range(6):
                prod = ops.rotate_add(prod, LANES << i)             # the head's 64 channels summed
            folded = ops.items(ops.mac([(prod, self.row0_both)]))    # ... kept at channel position 0
            del prod
            dense.update(self._pack_keys(dict(zip(pairs, folded)), group))
        D = ops.batch([dense[c] for c in range(CTS)])
        return ops.add(D, ops.conj(D))

    def _fold_keys(self, ct):
        """Sum over the 128 key positions of every (head, lane): the result at position 0."""

        ops = self.ops
        for i in range(6):
            ct = ops.rotate_add(ct, 8 << i)
        return ops.rotate_add(ct, HALF)

    def _spread_keys(self, ct):
        """Position 0 of every (head, lane) copied to all 128 key positions (other positions 0)."""

        ops = self.ops
        for i in range(6):
            ct = ops.rotate_add(ct, -(8 << i))
        return ops.rotate_add(ct, -HALF)

    def softmax(self, S2):
        """Alg2 at k = 1 on the dense scores (2 S): probabilities at the same positions, 0 off the
        causal set.  The row mean of the valid scores is subtracted first (softmax is invariant to
        it): the row sums over the n valid keys then satisfy 1 <= R / n <= n, a range one
        inverse-square-root series covers."""

        ops = self.ops
        # D also holds the non-causal scores of the diagonal block (c' = c, key lane > t): only the
        # valid ones enter the mean, and the series input is masked to the valid set
        mean = self._fold_keys(ops.mac([(S2, self.valid_over_n)]))       # 2 mean at position 0
        mean = self._spread_keys(ops.mac([(mean, self.row0)]))           # at every key position
        S2 = ops.sub(ops.adjust(S2, ops.limbs(mean), ops.scale(mean)), mean)
        self._mark("attention_mean")
        # the affine map lands on the prime of the next level: the series input's exact scale
        x = ops.mac([(S2, self.exp_alpha_valid)], out_scale=ops.ideal_scale(ops.limbs(S2) - 1))
        x = ops.add_const(x, self.exp_beta) if self.exp_beta else x
        x = self._refreshed_series_input(x, "exp")
        y = ops.poly(x, self.polys.exp)
        # invalid positions hold x = beta: remove the public E(0) there (no level)
        y = ops.add_vec(y, SlotConst(-self.exp_at_zero * self.invalid.value))
        rows = self._fold_keys(ops.mul(y, y))                            # R at (h, 0, t)
        rows = ops.items(ops.rotate(rows, [-8 * c for c in range(CTS)]))  # one launch, a rotation per item
        packed = ops.mac([(rows[c], self.rowc[c]) for c in range(CTS)])
        z = ops.mac([(packed, self.rs_in)], out_scale=ops.ideal_scale(ops.limbs(packed) - 1))
        z = ops.add_vec(z, self.rs_shift)                # slots outside the packed rows stay at 0
        z = self._refreshed_series_input(z, "rsqrt")
        lam = ops.poly(z, self.polys.rsqrt)             # rsqrt(R / n) at (h, c, t)
        spread = ops.batch(ops.rotate_offsets(lam, [8 * c for c in range(CTS)]))
        lam_c = self._spread_keys(ops.mac([(spread, self.inv_sqrt_count)]))   # 1 / sqrt(R) everywhere
        yl = ops.mul(y, lam_c)
        return ops.mul(yl, yl)

    def _refreshed_series_input(self, x, which: str):
        """With refresh_series_inputs: a two-pass refresh of a series input (|x| <= 1), then one
        scalar product that puts it back on its level's prime (the series' exact-scale chain)."""

        if not self.refresh_series_inputs:
            return x
        ops = self.ops
        self._mark("attention_softmax")
        self._tap(f"{which}_in", x)
        passes = self.spec.rsqrt_refresh_iterations if which == "rsqrt" else self.spec.exp_refresh_iterations
        x = self._tap(which, ops.refresh(x, bound_bits=0, program=self.series_programs.get(which), iterations=passes))
        self._mark(f"attention_{which}_refresh")
        lim = ops.limbs(x) - 1
        return ops.adjust(x, lim, ops.ideal_scale(lim))

    def pv(self, P, V):
        """sum_k P[h][q][k] Vz(k) for every query ciphertext: complex feature-major outputs.  The
        probability columns of pair (c, p) (key p in the lower half, key p + split(c) in the upper)
        reach channel position 0 by a giant rotation by 64 a (the 16 ciphertexts times their a, one
        batch) and a baby rotation by 8 b (one batch of all pairs); they are masked there, spread
        over the 64 channels and multiplied by the value carriers of both keys; the products of a
        query ciphertext are summed before one relinearisation, and the upper half's sum is
        added to the lower half's."""

        ops = self.ops
        if ops.limbs(P) > PV_INPUT_LIMBS:
            # the column mask, the product, W_O and the residual need no more: the rest of the
            # layer's work runs on fewer limbs (the residual is refreshed after it)
            P = ops.drop(P, PV_INPUT_LIMBS)
        if ops.limbs(V) > ops.limbs(P):
            V = ops.drop(V, ops.limbs(P))                 # the carriers only need P's level
        v_lo, v_up = self._lane_carriers(V, (0, self.lane[False]), (HALF, self.lane[True]))
        p_items = ops.items(P)
        giants = [(c, a) for c in range(CTS) for a in range((split(c) + LANES - 1) // LANES)]
        at = {k: i for i, k in enumerate(giants)}
        g_items = ops.items(ops.rotate(ops.batch([p_items[c] for c, _ in giants]), [64 * a for _, a in giants]))
        src = ops.batch([g_items[at[(c, p // LANES)]] for c, p in self.pairs])
        del g_items
        col = ops.rotate(src, [LANES * (p % LANES) for _, p in self.pairs])
        del src
        col = ops.mac([(col, self.row0_both)])
        for i in range(6):
            col = ops.rotate_add(col, -(LANES << i))      # within each half's heads
        right = self._pair_carriers(v_lo, v_up, self.pairs)
        sums = ops.mul_sum(col, right, [split(c) for c in range(CTS)])
        return ops.add(sums, ops.rotate(sums, HALF))

    def _tap(self, name, ct):
        if self._taps is not None:
            self._taps[name] = ct
        return ct

    def forward(self, A, V, mark=None, taps: dict | None = None):
        """Attention output and its intermediates; ``mark(name)`` (optional) is called after the
        scores, around each series-input refresh, and after the softmax and PV (stage timing);
        ``taps`` (optional) receives each series refresh's input and output."""

        self._mark = mark if mark is not None else (lambda name: None)
        self._taps = taps
        try:
            S2 = self.scores(A)
            self._mark("attention_scores")
            P = self.softmax(S2)
            self._mark("attention_softmax")
            out = self.pv(P, V)
            self._mark("attention_pv")
        finally:
            self._mark = lambda name: None
            self._taps = None
        return out, {"scores": S2, "probs": P}


def attention_input_numpy(xn: np.ndarray, spec: PrefillSpec, w: DecodeWeights) -> tuple[np.ndarray, np.ndarray]:
    """The slot vectors of the projection batch A (before RoPE) and the value batch V ([16, slots] complex)
    for a normalised input (gamma applied): what the GPU projections produce, for simulations."""

    from .layouts import FeatureMajorPrefillLayout

    lay = FeatureMajorPrefillLayout()
    xa = xn @ qk_matrix(w).T          # [128, 4096] complex channels
    xv = xn @ v_matrix(w).T
    A = np.asarray(lay.pack(xa.real)) + 1j * np.asarray(lay.pack(xa.imag))
    Vs = np.asarray(lay.pack(xv.real)) + 1j * np.asarray(lay.pack(xv.imag))
    return A, Vs


# ---------------------------------------------------------------------------- the GPU layer
def attention_key_rotations(spec: PrefillSpec, config) -> tuple[int, ...]:
    from .layouts import FeatureMajorPrefillLayout
    from .linear import bsgs_rotations
    from .norm import rmsnorm_rotations

    lay = FeatureMajorPrefillLayout()
    plan = config.plan(dimension=spec.hidden_dim, token_lanes=lay.tokens_per_cipher)
    rots = set(attention_rotations()) | set(bsgs_rotations(plan, config.hoist_strategy))
    rots |= set(rmsnorm_rotations(lay))
    return tuple(sorted(rots))


def prefill_key_rotations(spec: PrefillSpec, config, mlp_spec, bootstrap_spec, log_n: int = 16) -> tuple[int, ...]:
    """Every rotation key of one prefill layer: attention, projections, RMSNorm, the MLP block, the
    refresh and the conjugation."""

    from .bootstrap import requirements
    from .layouts import FeatureMajorPrefillLayout
    from .mlp import FeatureMajorMLPBlock

    rots = set(attention_key_rotations(spec, config))
    rots |= set(FeatureMajorMLPBlock.rotations(mlp_spec, FeatureMajorPrefillLayout(), config))
    rots |= set(requirements(bootstrap_spec, log_n).rotations)
    rots.add((1 << (log_n + 1)) - 1)
    return tuple(sorted(r for r in rots if r))


class PrefillLayer:
    """One encrypted prefill layer on the GPU: RMSNorm1, projections A and V (one baby-rotation set
    for both), RoPE, the attention core, W_O, the residual, one two-pass refresh of the residual,
    the MLP block and the second residual.

    ``steady``: the layer as it runs inside the model (the reference's layer_idx > 0 schedule,
    llama3fhe/graph/prefill.py:217-221,392-459): its input is the previous layer's output at a low
    level, so it is refreshed first (two passes, as one batch), and the attention refreshes the exp
    series' input (16 ciphertexts) and the inverse square root's (one packed ciphertext).  Without
    it the layer is the model's first, fed by a fresh encryption at the top of the chain."""

    def __init__(self, ctx, weights: DecodeWeights, spec: PrefillSpec | None = None, *, program, config=None,
                 mlp_spec=None, steady: bool = False, programs: dict | None = None):
        from .decode import CipherOps
        from .layouts import FeatureMajorPrefillLayout
        from .linear import LinearOperator, LinearWeight
        from .mlp import FeatureMajorMLPBlock, default_config
        from .norm import rmsnorm_coefficients

        self.ctx = ctx
        self.spec = PrefillSpec() if spec is None else spec
        self.spec.validate()
        self.layout = FeatureMajorPrefillLayout()
        self.config = default_config() if config is None else config
        self.ops = CipherOps(ctx, program)
        self.program = program
        self.steady = bool(steady)
        self.levels: dict = {}   # limbs at the stage boundaries of the last forward
        # refresh programs per site ("residual", "input", "exp", "rsqrt"); missing ones use ``program``
        self.programs = dict(programs or {})
        self.attn = PrefillAttention(self.ops, self.spec, refresh_series_inputs=self.steady,
                                     series_programs={k: self.programs[k] for k in ("exp", "rsqrt")
                                                      if k in self.programs})
        self.rms = rmsnorm_coefficients(self.spec.rms_degree, self.spec.rms_interval, self.spec.eps)
        self.op = LinearOperator(crypto_context=ctx, token_lanes=LANES, config=self.config)
        gamma = np.asarray(weights.input_layernorm, dtype=np.float64)
        qk = qk_matrix(weights, gamma)
        vm = v_matrix(weights, gamma)
        wo = wo_matrix(weights)
        self.w_qk = LinearWeight(np.ascontiguousarray(qk.real), crypto_context=ctx, imag=np.ascontiguousarray(qk.imag))
        self.w_v = LinearWeight(np.ascontiguousarray(vm.real), crypto_context=ctx, imag=np.ascontiguousarray(vm.imag))
        self.w_o = LinearWeight(np.ascontiguousarray(wo.real), crypto_context=ctx, imag=np.ascontiguousarray(wo.imag))
        self.mlp_spec = prefill_mlp_spec(self.spec) if mlp_spec is None else mlp_spec
        self.mlp = FeatureMajorMLPBlock(ctx, weights.gate_proj, weights.up_proj, weights.down_proj,
                                        norm_weight=weights.post_attention_layernorm, spec=self.mlp_spec,
                                        layout=self.layout, config=self.config, bootstrap_program=None)

    def forward(self, x_cts, taps: dict | None = None):
        """Layer output (16 ciphertexts) and the seconds of each stage.  ``taps``, when given,
        receives named intermediates (each refresh's input and output among them), so the error
        each stage adds can be measured by decryption."""

        import torch

        from . import fhe
        from .norm import rmsnorm_fhe

        ctx, ops = self.ctx, self.ops
        t: dict = {}
        t0 = time.perf_counter()

        def mark(name):
            nonlocal t0
            torch.cuda.synchronize()
            now = time.perf_counter()
            t[name] = t.get(name, 0.0) + now - t0
            t0 = now

        def tap(name, ct):
            if taps is not None:
                taps[name] = ct
            return ct

        x_cts = tuple(x_cts)
        if self.steady:
            xb = tap("input_in", ops.batch(x_cts))
            x_cts = tuple(ops.items(tap("input", ops.refresh(xb, bound_bits=self.spec.input_bound_bits,
                                                             program=self.programs.get("input"),
                                                             iterations=self.spec.input_refresh_iterations))))
            mark("refresh_input")
        xn = rmsnorm_fhe(x_cts, None, coeffs=self.rms, layout=self.layout, crypto_context=ctx).outputs
        mark("rmsnorm1")
        prepared = self.op.prepare(xn, self.spec.hidden_dim)
        a_out, _ = self.op.apply(xn, self.w_qk, prepared=prepared)
        v_out, _ = self.op.apply(xn, self.w_v, prepared=prepared)
        del prepared
        mark("qkv_projection")
        A, V = ops.batch(a_out), ops.batch(v_out)
        self.levels = {"input": ops.limbs(x_cts[0]), "rmsnorm1": ops.limbs(xn[0]), "A": ops.limbs(A)}
        out, _ = self.attn.forward(A, V, mark=mark, taps=taps)
        self.levels["attention"] = ops.limbs(out)
        t["attention"] = sum(v for k, v in t.items() if k.startswith("attention_"))
        proj, _ = self.op.apply(ops.items(out), self.w_o)
        delta = ops.batch(proj)
        delta = ops.add(delta, ops.conj(delta))
        x = fhe.pack_cipher_batch(list(x_cts))
        x = ops.adjust(x, ops.limbs(delta), ops.scale(delta))
        h = ops.add(x, delta)
        mark("w_o_residual")
        self.levels["residual"] = ops.limbs(h)
        tap("residual_in", h)
        h = tap("residual", ops.refresh(h, bound_bits=self.spec.residual_bound_bits,
                                        program=self.programs.get("residual"),
                                        iterations=self.spec.residual_refresh_iterations))
        mark("refresh")
        m_out, _ = self.mlp.forward(ops.items(h))
        m = tap("mlp", ops.batch(m_out))
        h2 = ops.adjust(h, ops.limbs(m), ops.scale(m))
        out = tap("output", ops.add(h2, m))
        self.levels["output"] = ops.limbs(out)
        ops.finish()
        mark("mlp_residual")
        return tuple(ops.items(out)), t


def setup_prefill_layer(client, ctx, weights: DecodeWeights, spec: PrefillSpec | None = None, config=None,
                        steady: bool = False):
    """Every rotation key of the layer and its refresh program, then the layer (``client`` holds
    the secret key; the layer itself only sees ``ctx``); ``steady`` as for ``PrefillLayer``."""

    from .bootstrap import generate
    from .mlp import default_config

    spec = PrefillSpec() if spec is None else spec
    config = default_config() if config is None else config
    bspec = prefill_bootstrap_spec()
    rots = prefill_key_rotations(spec, config, prefill_mlp_spec(spec), bspec, int(ctx.logN))
    client.generate_rotation_keys(rots)
    program = generate(ctx, bspec)
    programs = {k: generate(ctx, prefill_bootstrap_spec(r)) for k, r in refresh_raise_limbs(ctx.q_primes).items()}
    return PrefillLayer(ctx, weights, spec, program=program, config=config, steady=steady, programs=programs), rots
