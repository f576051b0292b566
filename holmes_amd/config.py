"""CKKS run configuration with the fields of llama3fhe/config.py:15-42 (``SimulatorConfig``),
defaults set for the MI355X FP64 arithmetic path (50-bit primes, scale 2^40)."""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path


@dataclass
class SimulatorConfig:
    logN: int = 16
    maxLevelsRemaining: int = 23
    level_budget: tuple[int, int] = (4, 4)
    dnum: int = 3
    dcrtBits: int = 50
    firstMod: int = 50
    secretKeyDist: str = "SPARSE_TERNARY"
    rescaleTech: str = "FIXEDMANUAL"
    device: str = "cuda"
    scaleBits: int = 40

    def rescale_policy(self) -> str:
        value = str(self.rescaleTech).lower()
        if value in {"fixedmanual", "fixed_manual", "manual"}:
            return "manual"
        if value in {"fixedauto", "fixed_auto", "auto"}:
            return "auto"
        raise ValueError(f"unsupported rescale policy: {value!r}")

    def validate(self) -> None:
        if int(self.logN) <= 1:
            raise ValueError("simulator.logN must be greater than one.")
        if int(self.maxLevelsRemaining) <= 0:
            raise ValueError("simulator.maxLevelsRemaining must be positive.")
        if int(self.dnum) <= 0 or int(self.dcrtBits) <= 0 or int(self.firstMod) <= 0:
            raise ValueError("simulator dnum/modulus parameters must be positive.")
        self.rescale_policy()

    @classmethod
    def from_json(cls, path: str | Path) -> "SimulatorConfig":
        sim = json.loads(Path(path).read_text(encoding="utf-8")).get("simulator", {})
        cfg = cls(**{k: (tuple(v) if k == "level_budget" else v) for k, v in sim.items() if k in cls.__dataclass_fields__})
        cfg.validate()
        return cfg


__all__ = ["SimulatorConfig"]
