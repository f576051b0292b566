"""Encrypted Llama-3 MLP block in the feature-major layout (llama3fhe/operators/linear/prefill/
mlp.py:37-135,373-519,723-1355; norm/rmsnorm.py; nonlinear/elementwise.py).

    y   = RMSNorm(x)                    (polynomial inverse square root, gamma folded into gate/up)
    g_p = y W_gate[p]^T,  u_p = y W_up[p]^T      for every 4096-feature page p of the 14336 features
    h_p = SiLU(g_p) * u_p               (SiLU a Chebyshev series on an interval)
    out = sum_p h_p W_down[:, p]^T
    out = 2^r * Bootstrap(2^-r * out)   (optional; the refresh a layer pipeline continues from)

Pages follow the reference's FeatureMajorMLPLayout: the intermediate width is cut into pages of
hidden_dim features, each page laid out like the canonical activation (16 ciphertexts for 128
tokens), the last page zero-padded.  Every projection is a 4096 x 4096 BSGS product of this
backend's LinearOperator, all projections of one input sharing its baby rotations.

With ``paired`` (the reference's carrier algebra, mlp.py:440-519) adjacent token ciphertexts are
paired as z = x_a + i x_b, and each page is one complex projection A = (gate + i up) / 4 applied to
z and conj(z): gate_half = z A^T + conj(conj(z) A^T) = z gate^T / 2, up_half = -i (z A^T -
conj(conj(z) A^T)) = z up^T / 2, and w + conj(w), -i (w - conj(w)) split each half into the two
tokens' real rows -- half the projection work of separate gate and up projections.  SiLU and the
product run on the real rows; their results are re-paired as h_a + i h_b, the down projection
(down / 2) runs on 8 complex ciphertexts per page, and out + conj(out), -i (out - conj(out)) give
the 16 real outputs.  The SiLU of all pages runs as one batch (each Paterson-Stockmeyer product one
batched key switch).

``mlp_block_numpy`` is the float64 oracle of the same arithmetic (the same polynomials), so the
decrypted output measures the encryption and key-switching error only.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import numpy as np

from . import fhe
from .context import CKKSContext
from .layouts import FeatureMajorPrefillLayout
from .linear import LinearOperator, LinearOperatorConfig, LinearWeight, bsgs_rotations
from .norm import rmsnorm_coefficients, rmsnorm_fhe, rmsnorm_numpy, rmsnorm_rotations
from .polynomial import chebyshev_coefficients, eval_chebyshev

def _items(ct, lo: int, hi: int):
    return ct.cipher_like([c[lo:hi] for c in ct.cv], batch_size=hi - lo)


__all__ = ["MLPBlockSpec", "FeatureMajorMLPBlock", "default_config", "mlp_block_numpy", "silu_coefficients"]


def silu_coefficients(degree: int = 63, interval=(-16.0, 16.0)) -> np.ndarray:
    """Chebyshev interpolant of x sigma(x) on ``interval`` (nonlinear/elementwise.py's SiLU)."""

    return chebyshev_coefficients(lambda x: x / (1.0 + np.exp(-x)), degree, interval)


@dataclass(frozen=True)
class MLPBlockSpec:
    hidden_dim: int = 4096
    intermediate_width: int = 14336
    silu_degree: int = 63
    silu_interval: tuple = (-16.0, 16.0)
    rms_degree: int = 15
    rms_interval: tuple = (0.5, 2.0)
    eps: float = 1e-5
    bootstrap_prescale_bits: int = 5      # |out| <= 2^5 before the refresh
    bootstrap_iterations: int = 2
    paired: bool = True                   # token ciphertexts paired as x + i y (the reference's carrier)

    @property
    def pages(self) -> int:
        return -(-int(self.intermediate_width) // int(self.hidden_dim))


def default_config() -> LinearOperatorConfig:
    """Baby step 64 (the reference's production plan, linear/config.py:123-134): the gate and up
    projections of every page share the inputs' 63 baby rotations, so a larger baby step trades
    shared rotations for 4x fewer giant rotations per projection."""

    return LinearOperatorConfig(baby_steps=64, baby_anchor_step=-1, max_plaintext_rows=512,
                                hoist_strategy="ext_double_hoist")


def _page(weight: np.ndarray, p: int, D: int, rows: bool) -> np.ndarray:
    """The D x D block of page p: gate/up rows p D .. (p + 1) D, down columns likewise."""

    out = np.zeros((D, D), dtype=np.float64)
    if rows:
        blk = weight[p * D:(p + 1) * D]
        out[:blk.shape[0]] = blk
    else:
        blk = weight[:, p * D:(p + 1) * D]
        out[:, :blk.shape[1]] = blk
    return out


def mlp_block_numpy(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                    norm_weight: np.ndarray | None = None, spec: MLPBlockSpec = MLPBlockSpec(), *,
                    exact: bool = False, functions: dict | None = None) -> np.ndarray:
    """float64 oracle of the block with the same polynomials (bootstrap excluded: exact);
    ``exact`` puts 1 / sqrt(m + eps) and x sigma(x) in place of the series (a textbook SwiGLU),
    ``functions`` ({"rms": f, "silu": g}) any other function in place of either series."""

    eps = float(spec.eps)
    fn = dict(functions or {})
    if exact:
        fn.setdefault("rms", lambda m: 1.0 / np.sqrt(m + eps))
        fn.setdefault("silu", lambda v: v / (1.0 + np.exp(-v)))
    rms = {"function": fn["rms"]} if "rms" in fn else rmsnorm_coefficients(spec.rms_degree, spec.rms_interval, eps)
    y = rmsnorm_numpy(x, norm_weight, rms)
    g = y @ np.asarray(gate, dtype=np.float64).T
    u = y @ np.asarray(up, dtype=np.float64).T
    if "silu" in fn:
        s = fn["silu"](g)
    else:
        a, b = spec.silu_interval
        s = np.polynomial.chebyshev.chebval((2.0 * g - (a + b)) / (b - a), silu_coefficients(spec.silu_degree,
                                                                                            spec.silu_interval))
    return (s * u) @ np.asarray(down, dtype=np.float64).T


class FeatureMajorMLPBlock:
    """The block's weights on the device (gamma folded into gate and up) and its schedule."""

    def __init__(self, ctx: CKKSContext, gate: np.ndarray, up: np.ndarray, down: np.ndarray, *,
                 norm_weight: np.ndarray | None = None, spec: MLPBlockSpec = MLPBlockSpec(),
                 layout: FeatureMajorPrefillLayout | None = None, config: LinearOperatorConfig | None = None,
                 bootstrap_program=None):
        D, Iw = int(spec.hidden_dim), int(spec.intermediate_width)
        if gate.shape != (Iw, D) or up.shape != (Iw, D) or down.shape != (D, Iw):
            raise ValueError(f"expected gate/up [{Iw}][{D}] and down [{D}][{Iw}]")
        self.ctx = ctx
        self.spec = spec
        self.layout = FeatureMajorPrefillLayout(seq_len=128, hidden_dim=D, slots=ctx.max_slots) if layout is None \
            else layout
        self.config = default_config() if config is None else config
        self.op = LinearOperator(crypto_context=ctx, token_lanes=self.layout.tokens_per_cipher, config=self.config)
        col = np.ones(D) if norm_weight is None else np.asarray(norm_weight, dtype=np.float64).reshape(-1)
        gate = np.asarray(gate, dtype=np.float64) * col[None, :]
        up = np.asarray(up, dtype=np.float64) * col[None, :]
        down = np.asarray(down, dtype=np.float64)
        if spec.paired:
            self.gate_up = [LinearWeight(0.25 * _page(gate, p, D, True), imag=0.25 * _page(up, p, D, True),
                                         crypto_context=ctx) for p in range(spec.pages)]
            self.down = [LinearWeight(0.5 * _page(down, p, D, False), crypto_context=ctx) for p in range(spec.pages)]
        else:
            self.gate = [LinearWeight(_page(gate, p, D, True), crypto_context=ctx) for p in range(spec.pages)]
            self.up = [LinearWeight(_page(up, p, D, True), crypto_context=ctx) for p in range(spec.pages)]
            self.down = [LinearWeight(_page(down, p, D, False), crypto_context=ctx) for p in range(spec.pages)]
        self.rms = rmsnorm_coefficients(spec.rms_degree, spec.rms_interval, spec.eps)
        self.silu = silu_coefficients(spec.silu_degree, spec.silu_interval)
        self.bootstrap_program = bootstrap_program

    @staticmethod
    def rotations(spec: MLPBlockSpec, layout: FeatureMajorPrefillLayout, config: LinearOperatorConfig | None = None) -> tuple:
        """Slot rotations the block uses (the bootstrap program's come from its requirements)."""

        config = default_config() if config is None else config
        plan = config.plan(dimension=int(spec.hidden_dim), token_lanes=layout.tokens_per_cipher)
        rots = set(bsgs_rotations(plan, config.hoist_strategy)) | set(rmsnorm_rotations(layout))
        if spec.paired:
            rots.add(4 * int(layout.slots) - 1)  # conjugation
        return tuple(sorted(rots))

    def _real(self, y, mark):
        """Separate gate and up projections per page on the real token ciphertexts."""

        ctx, spec = self.ctx, self.spec
        t0 = time.perf_counter()
        prep = self.op.prepare(y, spec.hidden_dim)
        gates, ups = [], []
        for p in range(spec.pages):
            gates += list(self.op.project(y, self.gate[p], prepared=prep))
            ups += list(self.op.project(y, self.up[p], prepared=prep))
        del prep
        t0 = mark("gate_up", t0)
        h = self._silu_product(fhe.pack_cipher_batch(gates), fhe.pack_cipher_batch(ups))
        t0 = mark("silu_product", t0)
        n = len(y)
        out = None
        for p in range(spec.pages):
            part = self.op.project([fhe.cipher_batch_item(h, p * n + i) for i in range(n)], self.down[p])
            out = list(part) if out is None else [fhe.homo_add(a, b, ctx) for a, b in zip(out, part)]
        mark("down", t0)
        return out

    def _silu_product(self, g, u):
        ctx, spec = self.ctx, self.spec
        s = eval_chebyshev(g, self.silu, ctx, interval=spec.silu_interval)
        u = fhe.align_to(u, u.state.replace(cur_limbs=int(s.state.cur_limbs)), ctx)
        return fhe.homo_mul_relin_rescale(s, u, ctx)

    def _paired(self, y, mark):
        """The reference's paired carrier: one complex gate + i up projection per page."""

        ctx, spec = self.ctx, self.spec
        n = len(y)
        if n % 2:
            raise ValueError("the paired MLP needs an even number of token ciphertexts")
        m = n // 2
        conj_g = ctx.M - 1
        t0 = time.perf_counter()
        yb = fhe.pack_cipher_batch(y)
        ya, yb_ = (fhe.pack_cipher_batch([fhe.cipher_batch_item(yb, i) for i in range(k, n, 2)]) for k in (0, 1))
        z = fhe.homo_add(ya, fhe.homo_mul_i(yb_, ctx), ctx)                  # x_a + i x_b, m items
        zz = fhe.pack_cipher_batch([z, fhe.homo_rotate(z, conj_g, ctx)])     # z and conj(z)
        inputs = [fhe.cipher_batch_item(zz, i) for i in range(2 * m)]
        prep = self.op.prepare(inputs, spec.hidden_dim)
        direct, ceval = [], []
        for p in range(spec.pages):
            outp = self.op.project(inputs, self.gate_up[p], prepared=prep)
            direct += list(outp[:m])
            ceval += list(outp[m:])
        del prep, inputs
        d = fhe.pack_cipher_batch(direct)
        cc = fhe.homo_rotate(fhe.pack_cipher_batch(ceval), conj_g, ctx)       # conj(conj(z) A^T)
        halves = fhe.pack_cipher_batch([fhe.homo_add(d, cc, ctx),            # z gate^T / 2
                                        fhe.homo_mul_i(fhe.homo_sub(d, cc, ctx), ctx, negative=True)])  # z up^T / 2
        hc = fhe.homo_rotate(halves, conj_g, ctx)
        re = fhe.homo_add(halves, hc, ctx)                                    # x_a rows: gate | up
        im = fhe.homo_mul_i(fhe.homo_sub(halves, hc, ctx), ctx, negative=True)  # x_b rows: gate | up
        k = spec.pages * m
        g = fhe.pack_cipher_batch([_items(re, 0, k), _items(im, 0, k)])
        u = fhe.pack_cipher_batch([_items(re, k, 2 * k), _items(im, k, 2 * k)])
        del d, cc, halves, hc, re, im
        t0 = mark("gate_up", t0)
        h = self._silu_product(g, u)                                           # [x_a rows | x_b rows]
        hz = fhe.homo_add(_items(h, 0, k), fhe.homo_mul_i(_items(h, k, 2 * k), ctx), ctx)  # re-paired
        t0 = mark("silu_product", t0)
        out = None
        for p in range(spec.pages):
            part = self.op.project([fhe.cipher_batch_item(hz, p * m + j) for j in range(m)], self.down[p])
            out = list(part) if out is None else [fhe.homo_add(a, b, ctx) for a, b in zip(out, part)]
        o = fhe.pack_cipher_batch(out)
        oc = fhe.homo_rotate(o, conj_g, ctx)
        even = fhe.homo_add(o, oc, ctx)
        odd = fhe.homo_mul_i(fhe.homo_sub(o, oc, ctx), ctx, negative=True)
        res = []
        for j in range(m):
            res += [fhe.cipher_batch_item(even, j), fhe.cipher_batch_item(odd, j)]
        mark("down", t0)
        return res

    def forward(self, x_cts):
        """Outputs (one ciphertext per input) and the seconds of each stage."""

        import torch

        from . import bootstrap as bs

        ctx, spec = self.ctx, self.spec
        t: dict = {}

        def mark(name, t0):
            torch.cuda.synchronize()
            t[name] = time.perf_counter() - t0
            return time.perf_counter()

        t0 = time.perf_counter()
        y = rmsnorm_fhe(x_cts, None, coeffs=self.rms, layout=self.layout, crypto_context=ctx).outputs
        t0 = mark("rmsnorm", t0)
        if spec.paired:
            out = self._paired(y, mark)
        else:
            out = self._real(y, mark)
        t0 = time.perf_counter()
        if self.bootstrap_program is not None:
            # the outputs refreshed as one batch: 2^-r (one scalar product + rescale), the
            # bootstrap (every key switch over all items), 2^r as an integer
            r = int(spec.bootstrap_prescale_bits)
            c = fhe.pack_cipher_batch(out)
            limbs = int(c.state.cur_limbs)
            enc = fhe.encode_scalar(2.0 ** -r, cur_limbs=limbs, scale_degree=1,
                                    scaling_factor=float(ctx.rescale_divisor_at(limbs)), context=ctx)
            small = fhe.homo_mul_scalar_rescale(c, enc, ctx)
            small = small.cipher_like(small.cv, state=small.state.replace(scaling_factor=c.state.scaling_factor))
            fresh = bs.bootstrap_with_correction(small, ctx, self.bootstrap_program,
                                                 iterations=int(spec.bootstrap_iterations), precision_bits=12)
            back = fhe.encode_scalar(1 << r, cur_limbs=int(fresh.state.cur_limbs), scale_degree=0, mode="integer",
                                     context=ctx)
            fresh = fhe.homo_mul_scalar(fresh, back, ctx)
            out = [fhe.cipher_batch_item(fresh, i) for i in range(fresh.batch_size)]
            t0 = mark("bootstrap", t0)
        return tuple(out), t
