"""CKKS run configuration with the field names and defaults of llama3fhe/config.py:15-42
(``SimulatorConfig``): depth 37, 59-bit primes with a 60-bit first modulus, dnum 3 -- a
default-constructed configuration builds the reference's chain (on this backend's 64-bit integer
path).  ``scaleBits`` is this backend's addition: the fixed scale 2^scaleBits, 0 meaning 2^dcrtBits
(the reference's fixed scale follows dcrtBits).  Both rescale techniques of the reference map onto
a policy name: FIXEDMANUAL -> "manual", FIXEDAUTO -> "auto".
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
    maxLevelsRemaining: int = 37
    level_budget: tuple[int, int] = (4, 4)
    dnum: int = 3
    dcrtBits: int = 59
    firstMod: int = 60
    secretKeyDist: str = "SPARSE_TERNARY"
    rescaleTech: str = "FIXEDMANUAL"
    device: str = "cuda"
    scaleBits: int = 0

    def scale_bits(self) -> int:
        """log2 of the fixed scale: scaleBits, or dcrtBits when scaleBits is 0."""

        return int(self.scaleBits) if int(self.scaleBits) else int(self.dcrtBits)

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
