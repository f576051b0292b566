"""CKKS run configuration with the field names of llama3fhe/config.py:15-42 (``SimulatorConfig``).

Field names are the interface (configuration files and callers set them by name); the defaults are
set for this backend's FP64 arithmetic path (50-bit primes, scale 2^40).  Both rescale techniques
of the reference map onto a policy name: FIXEDMANUAL -> "manual", FIXEDAUTO -> "auto".
"""

from __future__ import annotations

import json
from dataclasses import dataclass, fields
from pathlib import Path

_POLICY_ALIASES = {
    "manual": ("fixedmanual", "fixed_manual", "manual"),
    "auto": ("fixedauto", "fixed_auto", "auto"),
}


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
        """"manual" or "auto" for the configured rescale technique."""

        tech = str(self.rescaleTech).strip().lower()
        for policy, spellings in _POLICY_ALIASES.items():
            if tech in spellings:
                return policy
        raise ValueError(f"rescaleTech {self.rescaleTech!r} is neither a FIXEDMANUAL nor a FIXEDAUTO spelling")

    def validate(self) -> None:
        """Raise ValueError on a configuration no context can be built from."""

        problems = []
        if int(self.logN) < 2:
            problems.append(f"logN={self.logN} (needs at least 2)")
        if int(self.maxLevelsRemaining) < 1:
            problems.append(f"maxLevelsRemaining={self.maxLevelsRemaining} (needs at least 1)")
        for name in ("dnum", "dcrtBits", "firstMod"):
            if int(getattr(self, name)) < 1:
                problems.append(f"{name}={getattr(self, name)} (needs at least 1)")
        if problems:
            raise ValueError("invalid simulator configuration: " + ", ".join(problems))
        self.rescale_policy()

    @classmethod
    def from_json(cls, path: str | Path) -> "SimulatorConfig":
        """The ``simulator`` section of a model configuration file (unknown keys ignored)."""

        section = json.loads(Path(path).read_text(encoding="utf-8")).get("simulator", {})
        known = {f.name for f in fields(cls)}
        values = {k: v for k, v in section.items() if k in known}
        if "level_budget" in values:
            values["level_budget"] = tuple(values["level_budget"])
        cfg = cls(**values)
        cfg.validate()
        return cfg


__all__ = ["SimulatorConfig"]
