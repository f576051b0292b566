"""Execution-session boundary with the surface of llama3fhe/backend.py, backed by holmes_amd.

Holmes' operators reach their CKKS engine through one session object (``EasyFHEContext``: fields
``tensor, fhe, client, context, max_slots``; ``encrypt``, ``plaintext``, ``constant_bundle``,
``decrypt``, ``level_for_cipher``; llama3fhe/backend.py:249-397) and a handful of module helpers
(llama3fhe/backend.py:399-611).  Those names, arguments and the environment knobs the reference reads
are the interface kept here; every arithmetic call below them lands in libholmes_ckks (HIP, gfx950).

Constant caching is organised around a byte budget (``_Budget``) that the session's cache and the
bundles it hands out share:

* a bundle is admitted when its source arrays fit the per-source limit and the budget; admitted
  bundles are never evicted (layers scan their masks in the same order, so keeping the first ones
  is what makes the next layer hit);
* an admitted bundle asks the budget before it keeps an encoded plaintext; a plaintext that does
  not fit is returned to its caller and not kept, the bundle itself stays cached;
* a bundle that is not admitted never keeps anything (``cache_mode="none"``).

``tensor`` is PyTorch (ROCm): the easyfhe tensor shim's ``from_numpy``, ``empty``, ``zeros`` and
``cuda.Stream`` / ``Event`` / ``synchronize`` are torch's.
"""

from __future__ import annotations

import hashlib
import os
import re
import time
from dataclasses import dataclass, field
from math import log2

import numpy as np
import torch

from . import fhe
from .config import SimulatorConfig

# Constant names that differ only by decoder-layer index, or by the rank/iteration tag a benchmark
# prefixes, denote the same public mask and share one cache entry (llama3fhe/backend.py:23-54).
_NAME_RULES = (
    (re.compile(r"model\.layers\.\d+\."), "model.layers.*."),
    (re.compile(r"\.r\d+\.i\d+\."), ".r*.i*."),
)

# Environment knobs of the reference session (same names, same meaning).
ENV_CACHE_GB = "LLAMA_FHE_PLAIN_CACHE_GB"
ENV_CACHE_SOURCE_MB = "LLAMA_FHE_PLAIN_CACHE_MAX_SOURCE_MB"
ENV_STAGE_SYNC = "T2_STAGE_SYNC"
ENV_ALLOCATOR_TRIM = "LLAMA_FHE_ALLOCATOR_TRIM"

_STAT_FIELDS = ("entries", "bytes", "limit_bytes", "max_source_bytes", "hits", "misses", "skips")


def _normalized_constant_name(value: object) -> object:
    """Layer-independent form of a constant name (strings, or nested tuples / lists of them)."""

    if isinstance(value, str):
        for pattern, repl in _NAME_RULES:
            value = pattern.sub(repl, value)
        return value
    if isinstance(value, (list, tuple)):
        return tuple(map(_normalized_constant_name, value))
    return value


def _fingerprint(arrays: dict[str, np.ndarray]) -> str:
    """One digest over every named array's name, shape, dtype and bytes."""

    h = hashlib.sha256()
    for name in sorted(arrays):
        a = arrays[name]
        h.update(f"{name}|{a.shape}|{a.dtype.str}|".encode())
        h.update(memoryview(a).cast("B"))
    return h.hexdigest()


class _Budget:
    """Bytes a session may keep in cached constants."""

    def __init__(self, limit: int) -> None:
        self.limit = max(0, int(limit))
        self.used = 0

    def take(self, nbytes: int) -> bool:
        nbytes = int(nbytes)
        if self.used + nbytes > self.limit:
            return False
        self.used += nbytes
        return True

    def reset(self) -> None:
        self.used = 0


class SessionPlaintextCache:
    """Never-evicting constant cache under one byte budget (policy in the module docstring).

    ``get(key, factory, source_bytes=)`` returns the cached bundle for ``key`` or builds one with
    ``factory(admitted)``; ``transient(factory, source_bytes=)`` builds an uncached one.  Once
    ``clear()`` has run the cache refuses further use."""

    def __init__(self, *, limit_bytes: int, max_source_bytes: int) -> None:
        self._budget = _Budget(limit_bytes)
        self._max_source = max(0, int(max_source_bytes))
        self._bundles: dict[object, object] = {}
        self._stats = {"hits": 0, "misses": 0, "skips": 0}
        self._open = True

    # -- counters and limits (read-only views)
    limit_bytes = property(lambda self: self._budget.limit)
    max_source_bytes = property(lambda self: self._max_source)
    hits = property(lambda self: self._stats["hits"])
    misses = property(lambda self: self._stats["misses"])
    skips = property(lambda self: self._stats["skips"])
    closed = property(lambda self: not self._open)

    @property
    def budget(self) -> _Budget:
        return self._budget

    def accepts_source(self, source_bytes: int) -> bool:
        """True when a bundle of ``source_bytes`` source data may be cached at all."""

        return 0 < self._budget.limit and 0 <= int(source_bytes) <= self._max_source

    def _require_open(self) -> None:
        if not self._open:
            raise RuntimeError("the session plaintext cache was cleared and cannot be used again")

    def get(self, key, factory, *, source_bytes: int):
        self._require_open()
        if key in self._bundles:
            self._stats["hits"] += 1
            return self._bundles[key]
        self._stats["misses"] += 1
        admitted = self.accepts_source(source_bytes) and self._budget.take(source_bytes)
        bundle = factory(admitted)
        if admitted:
            self._bundles[key] = bundle
        else:
            self._stats["skips"] += 1
        return bundle

    def transient(self, factory, *, source_bytes: int):
        self._require_open()
        self._stats["misses"] += 1
        self._stats["skips"] += 1
        return factory(False)

    def info(self) -> dict[str, int]:
        values = (len(self._bundles), self._budget.used, self._budget.limit, self._max_source, self.hits,
                  self.misses, self.skips)
        return {k: int(v) for k, v in zip(_STAT_FIELDS, values)}

    def clear(self) -> None:
        self._open = False
        bundles, self._bundles = list(self._bundles.values()), {}
        self._budget.reset()
        for bundle in bundles:
            drop = getattr(bundle, "clear_cache", None)
            if callable(drop):
                drop()


def _cache_from_env() -> SessionPlaintextCache:
    gb = float(os.environ.get(ENV_CACHE_GB, "0") or 0)
    mb = float(os.environ.get(ENV_CACHE_SOURCE_MB, "1") or 0)
    return SessionPlaintextCache(limit_bytes=int(gb * 2**30), max_source_bytes=int(mb * 2**20))


@dataclass
class EasyFHEContext:
    """Session joining the client (keys, encrypt / decrypt) and the device context."""

    tensor: object
    fhe: object
    client: object
    context: object
    max_slots: int
    keygen_wall_time_s: float = 0.0
    plaintext_cache: SessionPlaintextCache = field(default_factory=_cache_from_env, init=False, repr=False)

    @property
    def device(self) -> str:
        return str(self.context.device)

    def _limbs_at(self, level: int) -> int:
        limbs = int(self.context.L) - int(level)
        if limbs < 1:
            raise ValueError(f"no limbs remain at level {level} of a {self.context.L}-limb chain")
        return limbs

    def level_for_cipher(self, cipher) -> int:
        return int(self.context.L) - int(cipher.state.cur_limbs)

    def configure_plaintext_cache(self, *, limit_bytes: int, max_source_bytes: int) -> None:
        """Replace the cache policy; only allowed while the cache is still untouched."""

        seen = self.plaintext_cache.info()
        if seen["entries"] or seen["misses"]:
            raise RuntimeError("configure the plaintext cache before the first constant is requested")
        self.plaintext_cache = SessionPlaintextCache(limit_bytes=limit_bytes, max_source_bytes=max_source_bytes)

    def encrypt(self, values: np.ndarray, *, level: int, slots: int | None = None):
        limbs = self._limbs_at(level)
        return self.client.encrypt(np.asarray(values).reshape(-1), device=self.device,
                                   slots=int(slots or self.max_slots), cur_limbs=limbs,
                                   scaling_factor=self.context.scale_at(limbs))

    def plaintext(self, values: np.ndarray, *, name: str, level: int, slots: int | None = None,
                  dtype: np.dtype = np.float64, is_ext: bool = False):
        limbs = self._limbs_at(level)
        bundle = self.constant_bundle({"value": np.asarray(values, dtype=dtype).reshape(-1)},
                                      cache_key=("vector", str(name)))
        state = fhe.CipherState(cur_limbs=limbs, scale_degree=1, scaling_factor=self.context.scale_at(limbs))
        return bundle.plaintext("value", state=state, slots=int(slots or self.max_slots), context=self.context,
                                is_ext=bool(is_ext))

    def constant_bundle(self, vectors: dict[str, np.ndarray], *, cache_key: object):
        """A ``fhe.ConstantBundle`` over ``vectors``: cached under (normalised ``cache_key``, content
        fingerprint) when the policy admits it, else built for this caller only."""

        arrays = {str(k): np.ascontiguousarray(v) for k, v in vectors.items()}
        nbytes = sum(a.nbytes for a in arrays.values())
        cache = self.plaintext_cache
        budget = cache.budget

        def build(admitted: bool):
            raws = {k: fhe.PackedRaw(torch.from_numpy(a)) for k, a in arrays.items()}
            if not admitted:
                return fhe.ConstantBundle(vectors=raws, cache_mode="none")
            return fhe.ConstantBundle(vectors=raws, cache_mode="plain", keep=budget.take)

        if not cache.accepts_source(nbytes):
            return cache.transient(build, source_bytes=nbytes)
        key = (_normalized_constant_name(cache_key), _fingerprint(arrays))
        return cache.get(key, build, source_bytes=nbytes)

    def plaintext_cache_info(self) -> dict[str, int]:
        return self.plaintext_cache.info()

    def clear_plaintext_cache(self) -> None:
        self.plaintext_cache.clear()

    def decrypt(self, cipher) -> np.ndarray:
        return np.asarray(self.client.decrypt(cipher)).reshape(-1)


# ---------------------------------------------------------------------------- module helpers
def plaintext_cache_snapshot(context) -> dict[str, int]:
    """The cache counters of ``context`` (zeros for an object without a cache)."""

    info = getattr(context, "plaintext_cache_info", None)
    if not callable(info):
        return dict.fromkeys(_STAT_FIELDS, 0)
    return {k: int(v) for k, v in info().items()}


def release_if_supported(value) -> None:
    """Free what ``value`` holds: its own ``release()``, else its constants' encoded cache."""

    for getter in (lambda v: getattr(v, "release", None),
                   lambda v: getattr(getattr(v, "constants", None), "clear_cache", None)):
        action = getter(value)
        if callable(action):
            action()
            return


def release_all(values) -> None:
    for value in values:
        release_if_supported(value)


def synchronize_device(device: str) -> None:
    dev = str(device)
    torch.cuda.synchronize(torch.device(dev) if dev.startswith("cuda") else None)


_stage_sync: list[bool | None] = [None]


def stage_sync_enabled() -> bool:
    """Stage boundaries synchronise the device unless T2_STAGE_SYNC=0 (llama3fhe/backend.py:450-487)."""

    if _stage_sync[0] is None:
        _stage_sync[0] = os.environ.get(ENV_STAGE_SYNC, "1") != "0"
    return bool(_stage_sync[0])


def set_stage_sync(enabled: bool | None) -> None:
    """Force stage synchronisation on or off (None: read the environment again)."""

    _stage_sync[0] = None if enabled is None else bool(enabled)


def profile_sync_device(device: str) -> None:
    if stage_sync_enabled():
        synchronize_device(device)


def trim_device_allocator_cache(device: str) -> None:
    """Return torch's cached device blocks to the driver when LLAMA_FHE_ALLOCATOR_TRIM=1."""

    if os.environ.get(ENV_ALLOCATOR_TRIM, "") == "1" and str(device).startswith("cuda"):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def cuda_memory_snapshot(device: str) -> dict[str, int | bool]:
    if not (str(device).startswith("cuda") and torch.cuda.is_available()):
        return {"available": False}
    dev = torch.device(str(device))
    free_b, total_b = torch.cuda.mem_get_info(dev)
    snap: dict[str, int | bool] = {"available": True}
    for name, fn in (("allocated", torch.cuda.memory_allocated), ("reserved", torch.cuda.memory_reserved),
                     ("peak_allocated", torch.cuda.max_memory_allocated),
                     ("peak_reserved", torch.cuda.max_memory_reserved)):
        snap[f"allocator_{name}_bytes"] = int(fn(dev))
    snap.update(device_used_bytes=int(total_b - free_b), device_free_bytes=int(free_b),
                device_total_bytes=int(total_b))
    return snap


def _power_of_two(value: int, name: str) -> int:
    value = int(value)
    if value < 1 or value & (value - 1):
        raise ValueError(f"{name} must be a power of two (got {value})")
    return value


def default_rotations(input_dim: int, block_out: int) -> set[int]:
    """Rotation set of an isolated operator test (llama3fhe/backend.py:540-553): the strides
    block_out 2^i below input_dim, and the powers of two below block_out."""

    d = _power_of_two(input_dim, "input_dim")
    b = _power_of_two(block_out, "block_out")
    return {b << i for i in range(d.bit_length() - 1)} | {1 << i for i in range(int(log2(b)))}


def create_sim_context(sim_cfg: SimulatorConfig, *, input_dim: int, block_out: int,
                       rotations=None, include_default_rotations: bool = True) -> EasyFHEContext:
    """Isolated-test session (llama3fhe/backend.py:556-596): context and keys for the requested
    rotations (plus the default set unless disabled)."""

    wanted = set(default_rotations(input_dim, block_out)) if include_default_rotations else set()
    wanted |= {int(r) for r in (rotations or ()) if int(r)}
    spec = fhe.CKKSContextSpec(
        depth=int(sim_cfg.maxLevelsRemaining), log_n=int(sim_cfg.logN), dnum=int(sim_cfg.dnum),
        dcrt_bits=int(sim_cfg.dcrtBits), first_mod=int(sim_cfg.firstMod),
        secret_key_dist=str(sim_cfg.secretKeyDist), scale_mode="fixed", rescale_policy=sim_cfg.rescale_policy(),
        rotations=tuple(sorted(wanted)), auto_load_keys=True, scale_bits=sim_cfg.scale_bits())
    t0 = time.perf_counter()
    client, context = fhe.generate_client_context(spec, device=str(sim_cfg.device))
    elapsed = time.perf_counter() - t0
    return EasyFHEContext(tensor=torch, fhe=fhe, client=client, context=context,
                          max_slots=int(context.max_slots), keygen_wall_time_s=float(elapsed))


__all__ = [
    "EasyFHEContext",
    "SessionPlaintextCache",
    "plaintext_cache_snapshot",
    "create_sim_context",
    "cuda_memory_snapshot",
    "default_rotations",
    "release_all",
    "release_if_supported",
    "synchronize_device",
    "profile_sync_device",
    "set_stage_sync",
    "stage_sync_enabled",
    "trim_device_allocator_cache",
]
