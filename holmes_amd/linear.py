"""Diagonal (BSGS) linear layers on the GPU: plan, weight, operator.

Restates the schedule of llama3fhe/operators/linear/config.py:47-380 (``LinearOperatorConfig``,
``LinearPlan``, ``LinearChunk``, ``linear_rotations``) and the execution of
llama3fhe/operators/linear/operator.py:203-467 (chunk loop, per-chunk giant steps, chunk-base
alignment rotation, accumulate, final rescale), re-organised for one GPU:

* the baby rotations of all inputs are computed once (one batched rotation per baby offset:
  every input shares that offset's key) and kept in HBM;
* a chunk's diagonals are packed and encoded on the GPU (``hck_pack_diagonals``,
  ``hck_encode``) and multiplied into every input at once by ``hck_bsgs_mac``
  (partial sums ``[2][G][inputs]``);
* each Horner giant step rotates all inputs' accumulators in one batched key switch with the
  shared giant key, as the batched giant step of bench/cmp/holmes_multi_mac.py:180-186.

Residues are exact: the result equals the oracle composition of the same rotations, MACs and
rescale bit for bit (tests/test_gpu_linear.py).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _native as nat
from . import fhe
from .context import Cipher, CipherState, CKKSContext, u64_cat

_HOIST_STRATEGIES = {"normal", "ext_normal", "ext_double_hoist"}


@dataclass(frozen=True)
class LinearChunk:
    index: int
    giant_base: int
    giant_count: int

    @property
    def name(self) -> str:
        return f"chunk.{int(self.index)}"


@dataclass(frozen=True)
class BabyBlock:
    start: int
    width: int


@dataclass(frozen=True)
class LinearPlan:
    """Physical BSGS schedule of one square block (llama3fhe/operators/linear/config.py:172-331)."""

    dimension: int
    token_lanes: int
    baby_steps: int
    baby_anchor_step: int
    max_plaintext_rows: int
    lane_shift: int = 0

    def __post_init__(self) -> None:
        if int(self.dimension) <= 0 or int(self.token_lanes) <= 0 or int(self.baby_steps) <= 0:
            raise ValueError("dimension, token_lanes and baby_steps must be positive.")
        if int(self.lane_shift) < 0:
            raise ValueError("lane_shift must be zero or positive.")
        if int(self.lane_shift) and int(self.lane_shift) * int(self.token_lanes) != int(self.dimension):
            raise ValueError("shifted-lane packing requires lane_shift * token_lanes == dimension.")
        if int(self.diagonals) % int(self.baby_steps):
            raise ValueError(f"baby_steps={self.baby_steps} must divide diagonals={self.diagonals}.")
        if int(self.baby_anchor_step) in (0, 1) or int(self.baby_anchor_step) < -1:
            raise ValueError("baby_anchor_step must be at least two or -1.")
        if int(self.max_plaintext_rows) < int(self.baby_steps):
            raise ValueError("max_plaintext_rows must hold one baby-step group.")

    @property
    def shifted_lanes(self) -> bool:
        return bool(int(self.lane_shift))

    @property
    def diagonals(self) -> int:
        return int(self.lane_shift) if self.shifted_lanes else int(self.dimension)

    @property
    def giant_steps(self) -> int:
        return int(self.diagonals) // int(self.baby_steps)

    @property
    def chunk_giants(self) -> int:
        return max(1, int(self.max_plaintext_rows) // int(self.baby_steps))

    @property
    def giant_offset(self) -> int:
        return int(self.baby_steps) * int(self.token_lanes)

    @property
    def baby_offsets(self) -> tuple[int, ...]:
        return tuple(b * int(self.token_lanes) for b in range(int(self.baby_steps)))

    @property
    def anchor_enabled(self) -> bool:
        return bool(int(self.baby_anchor_step) >= 2 and int(self.baby_steps) > int(self.baby_anchor_step))

    @property
    def baby_blocks(self) -> tuple[BabyBlock, ...]:
        width = int(self.baby_anchor_step) if self.anchor_enabled else int(self.baby_steps)
        return tuple(BabyBlock(start=s, width=min(width, int(self.baby_steps) - s))
                     for s in range(0, int(self.baby_steps), width))

    @property
    def baby_rotation_count(self) -> int:
        return max(0, int(self.baby_steps) - 1)

    @property
    def baby_key_offsets(self) -> tuple[int, ...]:
        width = int(self.baby_blocks[0].width)
        offsets = {s * int(self.token_lanes) for s in range(1, width)}
        if len(self.baby_blocks) > 1:
            offsets.add(int(self.baby_anchor_step) * int(self.token_lanes))
        return tuple(sorted(offsets))

    @property
    def fold_offsets(self) -> tuple[int, ...]:
        if not self.shifted_lanes:
            return ()
        return tuple(1 << i for i in range(int(self.token_lanes).bit_length() - 1))

    @property
    def lane_expand_offsets(self) -> tuple[int, ...]:
        if not self.shifted_lanes:
            return ()
        return tuple((int(self.dimension) - 1) * lane for lane in range(1, int(self.token_lanes)))

    @property
    def chunks(self) -> tuple[LinearChunk, ...]:
        return tuple(
            LinearChunk(index=i, giant_base=base, giant_count=min(self.chunk_giants, self.giant_steps - base))
            for i, base in enumerate(range(0, self.giant_steps, self.chunk_giants))
        )

    @property
    def chunk_sizes(self) -> tuple[int, ...]:
        return tuple(c.giant_count for c in self.chunks)

    @property
    def plaintext_chunks(self) -> int:
        return len(self.chunks)

    @property
    def cache_key(self) -> tuple[int, ...]:
        return (int(self.dimension), int(self.token_lanes), int(self.baby_steps), int(self.max_plaintext_rows),
                int(self.lane_shift))


@dataclass(frozen=True)
class LinearOperatorConfig:
    """Schedule knobs of one linear (llama3fhe/operators/linear/config.py:47-117)."""

    baby_steps: int = 32
    baby_anchor_step: int = 32
    max_plaintext_rows: int = 512
    reuse_baby_rotations: bool = True
    hoist_strategy: str = "normal"
    lane_shift: int = 0

    def __post_init__(self) -> None:
        if int(self.baby_steps) <= 0:
            raise ValueError("baby_steps must be positive.")
        if int(self.baby_anchor_step) in (0, 1) or int(self.baby_anchor_step) < -1:
            raise ValueError("baby_anchor_step must be at least two or -1.")
        if int(self.max_plaintext_rows) < int(self.baby_steps):
            raise ValueError("max_plaintext_rows must hold one baby-step group.")
        if str(self.hoist_strategy).lower() not in _HOIST_STRATEGIES:
            raise ValueError("hoist_strategy must be 'normal', 'ext_normal', or 'ext_double_hoist'.")

    def plan(self, *, dimension: int, token_lanes: int) -> LinearPlan:
        return LinearPlan(dimension=int(dimension), token_lanes=int(token_lanes), baby_steps=int(self.baby_steps),
                          baby_anchor_step=int(self.baby_anchor_step),
                          max_plaintext_rows=int(self.max_plaintext_rows), lane_shift=int(self.lane_shift))


def linear_rotations(*, dimension: int, token_lanes: int, slots: int | None = None,
                     include_conjugation: bool = False,
                     operator_config: LinearOperatorConfig | None = None) -> tuple[int, ...]:
    """Evaluation-key union of one schedule (llama3fhe/operators/linear/config.py:333-380)."""

    cfg = LinearOperatorConfig() if operator_config is None else operator_config
    plan = cfg.plan(dimension=int(dimension), token_lanes=int(token_lanes))
    rot = set(plan.baby_key_offsets)
    max_chunk = max(c.giant_count for c in plan.chunks)
    if max_chunk > 1:
        if str(cfg.hoist_strategy).lower() == "ext_double_hoist":
            rot.update(s * plan.giant_offset for s in range(1, int(max_chunk)))
        else:
            rot.add(plan.giant_offset)
    rot.update(int(c.giant_base) * plan.giant_offset for c in plan.chunks if int(c.giant_base))
    rot.update(plan.fold_offsets)
    rot.update(plan.lane_expand_offsets)
    if include_conjugation:
        if slots is None:
            raise ValueError("slots are required when conjugation is requested.")
        rot.add(4 * int(slots) - 1)
    return tuple(sorted(int(v) for v in rot if int(v)))


def bsgs_rotations(plan: LinearPlan, strategy: str = "normal") -> tuple[int, ...]:
    """Keys this GPU schedule uses: every baby offset, the giant offset (Horner) or every multiple
    of it inside a chunk (``ext_double_hoist``), the chunk bases."""

    rot = {o for o in plan.baby_offsets if o}
    if max(plan.chunk_sizes) > 1:
        if str(strategy).lower() == "ext_double_hoist":
            rot.update(s * plan.giant_offset for s in range(1, max(plan.chunk_sizes)))
        else:
            rot.add(plan.giant_offset)
    rot.update(int(c.giant_base) * plan.giant_offset for c in plan.chunks if int(c.giant_base))
    return tuple(sorted(rot))


class LinearWeight:
    """A square weight held on the device; packs and encodes one chunk's diagonals on demand.
    ``imag`` (same shape) makes the weight complex, weight + i imag: its diagonals are encoded as
    complex slots (the gate + i up projection of the paired MLP, llama3fhe/operators/linear/prefill/
    mlp.py:461-468)."""

    def __init__(self, weight: np.ndarray, *, crypto_context: CKKSContext, imag: np.ndarray | None = None):
        w = np.asarray(weight)
        if w.ndim != 2 or w.shape[0] != w.shape[1]:
            raise ValueError("LinearWeight expects a square matrix.")
        if imag is not None and np.asarray(imag).shape != w.shape:
            raise ValueError("the imaginary part must have the weight's shape")
        self.crypto_context = crypto_context
        self.dimension = int(w.shape[0])
        dev = crypto_context.device
        self._w = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float64)).to(dev)
        self._wi = None if imag is None else torch.from_numpy(np.ascontiguousarray(imag, dtype=np.float64)).to(dev)
        self._closed = False

    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def is_complex(self) -> bool:
        return self._wi is not None

    def plaintext(self, plan: LinearPlan, chunk: LinearChunk, *, limbs: int, scale: float,
                  flags: torch.Tensor | None = None) -> torch.Tensor:
        """Encoded diagonals [giant_count * baby_steps][limbs][N] of ``chunk`` (NTT domain).
        ``flags`` (int32, one per row) defers the overflow check to the caller."""

        if self._closed:
            raise RuntimeError("linear weight is closed")
        ctx = self.crypto_context

        def rows(w):
            return ctx.pack_diagonals(w, lanes=plan.token_lanes, lane_shift=plan.lane_shift,
                                      baby_steps=plan.baby_steps, giant_base=chunk.giant_base,
                                      giant_count=chunk.giant_count)

        if self._wi is None:
            return ctx.encode_real(rows(self._w), scale, limbs, flags=flags)
        return ctx.encode(rows(self._w), scale, limbs, values_im=rows(self._wi), flags=flags)

    def close(self) -> None:
        self._w = None
        self._wi = None
        self._closed = True


def _stack(ciphers) -> tuple[torch.Tensor, torch.Tensor, CipherState]:
    ciphers = tuple(ciphers)
    states = {(int(c.state.cur_limbs), int(c.state.scale_degree), float(c.state.scaling_factor)) for c in ciphers}
    if len(states) != 1:
        raise ValueError("linear inputs must enter at one common level and scale.")
    limbs = ciphers[0].state.cur_limbs
    c0 = u64_cat([c.cv[0][:, :limbs] for c in ciphers])
    c1 = u64_cat([c.cv[1][:, :limbs] for c in ciphers])
    return c0, c1, ciphers[0].state


class LinearOperator:
    """A reusable BSGS schedule over the ``token_lanes`` feature-major layout.  With
    ``config.lane_shift`` the input is in the shifted-lane packing of llama3fhe/layouts/
    shifted_lane.py:1-24 (lane l of channel c holds x[(c + lane_shift l) mod D]): the schedule has
    ``lane_shift`` diagonals and lane l of each output channel holds the partial product over the
    input block [lane_shift l, lane_shift (l + 1)); the caller folds the lanes."""

    def __init__(self, *, crypto_context, token_lanes: int, config: LinearOperatorConfig | None = None):
        self.crypto_context = crypto_context
        self.token_lanes = int(token_lanes)
        if self.token_lanes <= 0:
            raise ValueError("token_lanes must be positive.")
        self.config = LinearOperatorConfig() if config is None else config
        self._closed = False

    @property
    def closed(self) -> bool:
        return self._closed

    def plan(self, dimension: int) -> LinearPlan:
        return self.config.plan(dimension=int(dimension), token_lanes=self.token_lanes)

    def _ctx(self) -> CKKSContext:
        cc = self.crypto_context
        return getattr(cc, "context", cc)

    def _rotate_all(self, c0, c1, rotation: int, limbs: int, acc=None):
        ctx = self._ctx()
        g = ctx.galois_element(rotation)
        if acc is None:
            return ctx.rotate_raw(c0, c1, limbs, g, ctx.key_for_galois(g))
        # rotate-and-add in one pass, written over the addend
        return ctx.rotate_raw(c0, c1, limbs, g, ctx.key_for_galois(g), out0=acc[0], out1=acc[1], acc=acc)

    def prepare(self, input_ciphers, dimension: int):
        """The inputs stacked into one batch and their baby rotations (each offset one batched
        rotation over all inputs), for every projection of the same inputs to share."""

        inputs = tuple(input_ciphers)
        ctx = self._ctx()
        plan = self.plan(dimension)
        x0, x1, state = _stack(inputs)
        xc = Cipher([x0, x1], state, slots=inputs[0].slots)
        babies = fhe.prepare_hoisted_baby_rotations(xc, plan.baby_offsets, ctx,
                                                    strategy=str(self.config.hoist_strategy).lower(),
                                                    baby_anchor_step=int(plan.baby_anchor_step))
        return {"inputs": inputs, "stacked": xc, "babies": babies, "plan": plan.cache_key}

    def apply(self, input_ciphers, weight: LinearWeight, *, chunk_indices=None, rescale: bool = True,
              weight_scale: float | None = None, prepared: dict | None = None):
        """BSGS projection of every input; returns (outputs, stage_seconds).

        Weights are encoded at ``weight_scale`` (default: the prime the final rescale divides by,
        so the output returns to the input scale).  ``prepared`` (from ``prepare`` on the same
        inputs and dimension) reuses their baby rotations."""

        if self._closed:
            raise RuntimeError("linear operator is closed.")
        inputs = tuple(input_ciphers)
        if not inputs:
            return (), {}
        if weight.closed:
            raise RuntimeError("cannot apply a closed linear weight.")
        ctx = self._ctx()
        plan = self.plan(weight.dimension)
        chunks = plan.chunks if chunk_indices is None else tuple(plan.chunks[int(i)] for i in chunk_indices)
        if prepared is None:
            prepared = self.prepare(inputs, weight.dimension)
        elif prepared["plan"] != plan.cache_key or len(prepared["inputs"]) != len(inputs) or any(
                a is not b for a, b in zip(prepared["inputs"], inputs)):
            raise ValueError("prepared rotations belong to other inputs or another plan")
        xc, babies = prepared["stacked"], prepared["babies"]
        state = xc.state
        limbs = int(state.cur_limbs)
        if rescale and limbs < 2:
            raise ValueError("rescale needs at least two limbs")
        wscale = float(ctx.rescale_divisor_at(limbs)) if weight_scale is None else float(weight_scale)
        idx = ctx.q_prime_idx(limbs)
        strategy = str(self.config.hoist_strategy).lower()
        x0 = xc.cv[0]
        total0 = total1 = None
        # encode overflow flags of every chunk, read back once after the last chunk
        flags = torch.zeros(int(plan.max_plaintext_rows), dtype=torch.int32, device=x0.device)
        pt_state = CipherState(cur_limbs=limbs, scale_degree=1, scaling_factor=wscale)
        for chunk in chunks:
            pts = fhe.Plaintext(weight.plaintext(plan, chunk, limbs=limbs, scale=wscale, flags=flags), pt_state,
                                slots=xc.slots)
            res = fhe.hoisted_mac_sum(xc, plan.baby_offsets, pts, plan.giant_offset, int(chunk.giant_count), ctx,
                                      strategy=strategy, baby_anchor_step=int(plan.baby_anchor_step),
                                      baby_rotations=babies)
            del pts
            acc0, acc1 = res.cv
            base = int(chunk.giant_base) * plan.giant_offset
            if total0 is None:
                if base:
                    total0, total1 = self._rotate_all(acc0, acc1, base, limbs)
                else:
                    total0, total1 = acc0, acc1
            elif base:
                # chunk alignment rotation, accumulated into the running total in the same pass
                self._rotate_all(acc0, acc1, base, limbs, acc=(total0, total1))
            else:
                ctx.poly_op(nat.HCK_OP_ADD, total0, total0, acc0, prime_idx=idx)
                ctx.poly_op(nat.HCK_OP_ADD, total1, total1, acc1, prime_idx=idx)
            del res
        ctx.check_encode_flags(flags)
        out_state = state.replace(scale_degree=int(state.scale_degree) + 1,
                                  scaling_factor=float(state.scaling_factor) * wscale)
        slots = inputs[0].slots
        if rescale:
            both = ctx.rescale_raw(u64_cat([total0, total1]), limbs)
            n_in = total0.shape[0]
            total0, total1 = both[:n_in], both[n_in:]
            out_state = out_state.replace(cur_limbs=limbs - 1, scale_degree=int(state.scale_degree),
                                          scaling_factor=out_state.scaling_factor / float(ctx.rescale_divisor_at(limbs)))
        outputs = []
        start = 0
        for c in inputs:
            B = c.batch_size
            outputs.append(Cipher([total0[start:start + B], total1[start:start + B]], out_state, slots=slots))
            start += B
        return tuple(outputs), {}

    def project(self, input_ciphers, weight: LinearWeight, **kwargs):
        outputs, _ = self.apply(input_ciphers, weight, **kwargs)
        return outputs

    def close(self) -> None:
        self._closed = True


__all__ = ["LinearChunk", "BabyBlock", "LinearPlan", "LinearOperatorConfig", "linear_rotations",
           "bsgs_rotations", "LinearWeight", "LinearOperator"]
