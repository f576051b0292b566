"""The bootstrap operator Holmes' layers refresh through (llama3fhe/operators/nonlinear/bootstrap.py:
``BootstrapConfig`` 47-160, ``BootstrapOperator`` 163-470): one prepared full-slot program, an
optional deep program (a shallower CoeffToSlot / SlotToCoeff budget that leaves more levels) and
one sparse-slot program per period in ``sparse_log_slots``; ``refresh`` picks among them and runs
the one- or two-pass bootstrap of ``holmes_amd.bootstrap``.

A sparse program refreshes a message that is periodic with its period: the caller promises the
periodicity (``periodic_slots``), the ciphertext is viewed at that many slots (the same polynomial,
which lies in the period's subring) and viewed back at its own slot count afterwards.  A request
without a matching program is an error, never a silent dense refresh."""

from __future__ import annotations

import time
from dataclasses import dataclass, field

from . import bootstrap as bs

__all__ = ["BootstrapConfig", "BootstrapOperator"]


@dataclass(frozen=True)
class BootstrapConfig:
    log_slots: int = 15
    level_budget: tuple = (3, 3)
    output_levels: int = 0           # 0: every level the program leaves
    iterations: int = 2
    precision_bits: int = 12
    mode: str = "modraise_first"
    strategy: str = "double_hoist"
    dim1: tuple | None = None
    baby_step: tuple | None = None
    evict_rotation_cache: bool = False
    deep_level_budget: tuple | None = None
    deep_output_levels: int | None = None
    sparse_log_slots: int | tuple | None = None

    def __post_init__(self) -> None:
        if (self.deep_level_budget is None) != (self.deep_output_levels is None):
            raise ValueError("give deep_level_budget and deep_output_levels together (or neither)")
        ks = self.sparse_log_slots_tuple
        if len(ks) != len(set(ks)):
            raise ValueError(f"sparse_log_slots repeats an entry: {self.sparse_log_slots}")
        bad = [k for k in ks if not 0 < k < int(self.log_slots)]
        if bad:
            raise ValueError(f"sparse_log_slots entries must lie strictly between 0 and log_slots "
                             f"({self.log_slots}); got {bad}")

    @property
    def sparse_log_slots_tuple(self) -> tuple[int, ...]:
        v = self.sparse_log_slots
        if v is None:
            return ()
        return (int(v),) if isinstance(v, int) else tuple(int(k) for k in v)

    @property
    def sparse_slot_periods(self) -> tuple[int, ...]:
        return tuple(1 << k for k in self.sparse_log_slots_tuple)

    @property
    def sparse_slots(self) -> int | None:
        periods = self.sparse_slot_periods
        return periods[0] if periods else None

    def sparse_level_budget(self, log_slots: int | None = None) -> tuple[int, int] | None:
        """The main budget, each entry capped at the sparse program's layer count."""

        ks = self.sparse_log_slots_tuple
        if not ks:
            return None
        k = ks[0] if log_slots is None else int(log_slots)
        return tuple(min(int(b), k) for b in self.level_budget)

    def _spec(self, log_slots: int, budget, output_levels: int, fixed_babies: bool) -> bs.BootstrapSpec:
        return bs.BootstrapSpec(log_slots=int(log_slots), level_budget=tuple(int(b) for b in budget),
                                output_levels=int(output_levels), strategy=str(self.strategy), mode=str(self.mode),
                                dim1=self.dim1 if fixed_babies else None,
                                baby_step=self.baby_step if fixed_babies else None)

    def spec(self) -> bs.BootstrapSpec:
        return self._spec(self.log_slots, self.level_budget, self.output_levels, True)

    def sparse_specs(self) -> tuple[bs.BootstrapSpec, ...]:
        """One spec per ``sparse_log_slots`` entry, in that order (automatic baby steps: the fixed
        ones of the full program need not fit a smaller transform)."""

        return tuple(self._spec(k, self.sparse_level_budget(k), self.output_levels, False)
                     for k in self.sparse_log_slots_tuple)

    def sparse_spec(self) -> bs.BootstrapSpec | None:
        specs = self.sparse_specs()
        return specs[0] if specs else None

    def deep_spec(self) -> bs.BootstrapSpec | None:
        if self.deep_level_budget is None:
            return None
        return self._spec(self.log_slots, self.deep_level_budget, self.deep_output_levels, True)

    def all_specs(self) -> tuple[bs.BootstrapSpec, ...]:
        deep = self.deep_spec()
        return (self.spec(),) + (() if deep is None else (deep,)) + self.sparse_specs()


@dataclass
class BootstrapOperator:
    """Prepared programs plus the counters the reference's benches read."""

    crypto_context: object
    config: BootstrapConfig
    program: object
    setup_seconds: float
    deep_program: object | None = None
    sparse_programs: dict = field(default_factory=dict)   # {period slots: program}
    calls: int = 0
    native_calls: int = 0
    sparse_calls: int = 0

    @classmethod
    def prepare(cls, crypto_context, config: BootstrapConfig | None = None) -> "BootstrapOperator":
        """Plan every program of ``config`` on the context (its rotation keys must include
        ``bs.requirements(config.all_specs(), log_n).rotations``)."""

        config = BootstrapConfig() if config is None else config
        ctx = getattr(crypto_context, "context", crypto_context)
        t0 = time.perf_counter()
        program = bs.generate(ctx, config.spec())
        deep = config.deep_spec()
        deep_program = None if deep is None else bs.generate(ctx, deep)
        sparse = {spec.slots: bs.generate(ctx, spec) for spec in config.sparse_specs()}
        return cls(crypto_context=crypto_context, config=config, program=program, deep_program=deep_program,
                   sparse_programs=sparse, setup_seconds=time.perf_counter() - t0)

    @property
    def sparse_slot_periods(self) -> tuple[int, ...]:
        return tuple(sorted(self.sparse_programs))

    def has_sparse_program(self, period: int) -> bool:
        return int(period) in self.sparse_programs

    def refresh(self, cipher, *, iterations: int | None = None, precision_bits: int | None = None,
                use_deep_program: bool = False, periodic_slots: int | None = None, bound_bits: int = 0):
        """A refreshed copy of ``cipher`` (the input is not consumed)."""

        ctx = getattr(self.crypto_context, "context", self.crypto_context)
        program = self.program
        if use_deep_program:
            if self.deep_program is None:
                raise ValueError("a deep refresh needs deep_level_budget in the BootstrapConfig")
            program = self.deep_program
        full = int(cipher.slots)
        src = cipher
        if periodic_slots is not None:
            p = int(periodic_slots)
            if use_deep_program:
                raise ValueError("periodic_slots and use_deep_program exclude each other")
            program = self.sparse_programs.get(p)
            if program is None:
                raise ValueError(f"periodic_slots={p} has no sparse program (sparse_log_slots = "
                                 f"{self.config.sparse_log_slots})")
            if full % p:
                raise ValueError(f"a ciphertext of {full} slots cannot repeat with period {p}")
            src = cipher.cipher_like(cipher.cv, slots=p)
            self.sparse_calls += 1
        its = int(self.config.iterations if iterations is None else iterations)
        pb = int(self.config.precision_bits if precision_bits is None else precision_bits)
        out = bs.bootstrap_with_correction(src, ctx, program, iterations=its, precision_bits=pb,
                                           bound_bits=int(bound_bits))
        self.calls += 1
        self.native_calls += its
        if int(out.slots) != full:
            out = out.cipher_like(out.cv, slots=full)
        return out
