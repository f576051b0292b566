"""Writes tests/golden/easyfhe_surface.json: every ``easyfhe`` import and attribute that the
reference package llama3fhe uses, found by reading its sources as text (nothing is imported or run).

Run from the repository root in the container that holds /root/reference:
    python tests/golden/make_easyfhe_surface.py
The JSON is committed; tests/test_easyfhe_surface.py resolves every entry after
``holmes_amd.easyfhe_compat.install()``.
"""

from __future__ import annotations

import json
import re
import sys
from pathlib import Path

REF = Path("/root/reference/llama3fhe")
OUT = Path(__file__).resolve().parent / "easyfhe_surface.json"

IMPORT = re.compile(r"^\s*import (easyfhe[\w.]*)(?: as (\w+))?\s*$")
FROM = re.compile(r"^\s*from (easyfhe[\w.]*) import ([\w, ()]+)")
DOTTED = re.compile(r"\b(easyfhe(?:\.[A-Za-z_]\w*)+)")


def _attrs(text: str, alias: str) -> set[str]:
    return {m.group(1) for m in re.finditer(rf"\b{re.escape(alias)}\.([A-Za-z_][\w.]*)", text)}


def main() -> int:
    if not REF.is_dir():
        print(f"{REF} not found", file=sys.stderr)
        return 1
    modules: set[str] = set()
    names: set[tuple[str, str]] = set()
    dotted: set[str] = set()
    fhe_attrs: set[str] = set()
    bs_attrs: set[str] = set()
    shim_attrs: set[str] = set()
    files: list[str] = []
    for path in sorted(REF.rglob("*.py")):
        text = path.read_text(encoding="utf-8", errors="replace")
        if "easyfhe" not in text:
            continue
        files.append(str(path.relative_to(REF.parent)))
        for line in text.splitlines():
            m = IMPORT.match(line)
            if m:
                modules.add(m.group(1))
                if m.group(2) == "torch":
                    shim_attrs |= _attrs(text, "torch")
                elif m.group(2) == "bs":
                    bs_attrs |= _attrs(text, "bs")
                continue
            m = FROM.match(line)
            if m:
                for name in re.split(r"[,\s()]+", m.group(2)):
                    if name:
                        names.add((m.group(1), name))
        for m in DOTTED.finditer(text):
            if not m.group(1).endswith(("py", "cuda.Event(")):
                dotted.add(m.group(1))
        if re.search(r"^\s*from easyfhe import fhe", text, re.M):
            fhe_attrs |= {a.split(".")[0] for a in _attrs(text, "fhe")}
    # attribute chains on the tensor shim that are torch's own module paths stay whole
    surface = {
        "source": "llama3fhe/ (text search; see make_easyfhe_surface.py)",
        "files": files,
        "modules": sorted(modules),
        "from_imports": sorted([list(n) for n in names]),
        "dotted": sorted(dotted),
        "fhe_attributes": sorted(fhe_attrs),
        "bs_attributes": sorted({a.split(".")[0] for a in bs_attrs}),
        "shim_attributes": sorted(shim_attrs),
    }
    OUT.write_text(json.dumps(surface, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {OUT}: {len(modules)} modules, {len(names)} from-imports, {len(fhe_attrs)} fhe names")
    return 0


if __name__ == "__main__":
    sys.exit(main())
