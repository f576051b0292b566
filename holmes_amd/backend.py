"""Execution-session boundary with the surface of llama3fhe/backend.py, backed by holmes_amd.

Holmes' operators talk to their CKKS engine through ``EasyFHEContext`` (fields ``tensor, fhe,
client, context, max_slots``; methods ``encrypt, plaintext, constant_bundle, decrypt,
level_for_cipher``; llama3fhe/backend.py:249-397) and the module helpers of
llama3fhe/backend.py:399-611.  This module keeps those names, arguments and error behaviour so
operator code written against them runs on one MI355X with world size 1; every arithmetic call
lands in libholmes_ckks (HIP, gfx950).

``tensor`` is PyTorch (ROCm): the easyfhe tensor shim's ``from_numpy``, ``empty``, ``zeros``,
``cuda.Stream`` / ``Event`` / ``synchronize`` map onto torch's.
"""

from __future__ import annotations

import hashlib
import os
import re
import time
from collections import OrderedDict
from dataclasses import dataclass, field
from math import log2

import numpy as np
import torch

from . import fhe
from .config import SimulatorConfig

_LAYER_CACHE_NAME = re.compile(r"model\.layers\.\d+\.")
_RANK_ITER_CACHE_NAME = re.compile(r"\.r\d+\.i\d+\.")


def _normalized_constant_name(value: object) -> object:
    """Names that differ only by layer index or rank/iteration prefix share a cache entry
    (llama3fhe/backend.py:47-54)."""

    if isinstance(value, str):
        value = _LAYER_CACHE_NAME.sub("model.layers.*.", value)
        return _RANK_ITER_CACHE_NAME.sub(".r*.i*.", value)
    if isinstance(value, (tuple, list)):
        return tuple(_normalized_constant_name(item) for item in value)
    return value


def _array_digest(array: np.ndarray) -> str:
    return hashlib.blake2b(memoryview(np.ascontiguousarray(array)).cast("B"), digest_size=16).hexdigest()


class SessionPlaintextCache:
    """First-fit byte-capped cache of immutable constant bundles (llama3fhe/backend.py:129-247):
    an admitted entry is never evicted during a scan; an entry that would cross the budget stays
    transient for its caller."""

    def __init__(self, *, limit_bytes: int, max_source_bytes: int) -> None:
        self.limit_bytes = max(0, int(limit_bytes))
        self.max_source_bytes = max(0, int(max_source_bytes))
        self._entries: OrderedDict[object, fhe.ConstantBundle] = OrderedDict()
        self._bytes = 0
        self.hits = 0
        self.misses = 0
        self.skips = 0
        self.closed = False

    def accepts_source(self, source_bytes: int) -> bool:
        return self.limit_bytes > 0 and int(source_bytes) <= self.max_source_bytes

    def get(self, key, factory, *, source_bytes: int):
        if self.closed:
            raise RuntimeError("session plaintext cache is closed")
        hit = self._entries.get(key)
        if hit is not None:
            self.hits += 1
            return hit
        self.misses += 1
        admit = self.accepts_source(source_bytes) and self._bytes + int(source_bytes) <= self.limit_bytes
        bundle = factory(admit)
        if admit:
            self._entries[key] = bundle
            self._bytes += int(source_bytes)
        else:
            self.skips += 1
        return bundle

    def transient(self, factory, *, source_bytes: int):
        if self.closed:
            raise RuntimeError("session plaintext cache is closed")
        self.misses += 1
        self.skips += 1
        return factory(False)

    def info(self) -> dict[str, int]:
        return {
            "entries": len(self._entries),
            "bytes": int(self._bytes),
            "limit_bytes": int(self.limit_bytes),
            "max_source_bytes": int(self.max_source_bytes),
            "hits": int(self.hits),
            "misses": int(self.misses),
            "skips": int(self.skips),
        }

    def clear(self) -> None:
        for bundle in self._entries.values():
            clear_cache = getattr(bundle, "clear_cache", None)
            if callable(clear_cache):
                clear_cache()
        self._entries.clear()
        self._bytes = 0
        self.closed = True


@dataclass
class EasyFHEContext:
    """Data-only session joining the client and the device context."""

    tensor: object
    fhe: object
    client: object
    context: object
    max_slots: int
    keygen_wall_time_s: float = 0.0
    plaintext_cache: SessionPlaintextCache = field(init=False, repr=False)

    def __post_init__(self) -> None:
        limit_gb = float(os.environ.get("LLAMA_FHE_PLAIN_CACHE_GB", "0"))
        max_source_mb = float(os.environ.get("LLAMA_FHE_PLAIN_CACHE_MAX_SOURCE_MB", "1"))
        self.plaintext_cache = SessionPlaintextCache(
            limit_bytes=int(limit_gb * 1024**3), max_source_bytes=int(max_source_mb * 1024**2)
        )

    def configure_plaintext_cache(self, *, limit_bytes: int, max_source_bytes: int) -> None:
        info = self.plaintext_cache.info()
        if info["entries"] or info["misses"]:
            raise RuntimeError("plaintext cache policy must be fixed before first use")
        self.plaintext_cache = SessionPlaintextCache(limit_bytes=limit_bytes, max_source_bytes=max_source_bytes)

    @property
    def device(self) -> str:
        return str(self.context.device)

    def level_for_cipher(self, cipher) -> int:
        return int(self.context.L) - int(cipher.state.cur_limbs)

    def encrypt(self, values: np.ndarray, *, level: int, slots: int | None = None):
        cur_limbs = int(self.context.L) - int(level)
        if cur_limbs < 1:
            raise ValueError(f"level {level} leaves no limbs (L = {self.context.L})")
        return self.client.encrypt(
            np.asarray(values).reshape(-1),
            device=self.device,
            slots=self.max_slots if slots is None else int(slots),
            cur_limbs=cur_limbs,
            scaling_factor=self.context.scale_at(cur_limbs),
        )

    def plaintext(self, values: np.ndarray, *, name: str, level: int, slots: int | None = None,
                  dtype: np.dtype = np.float64, is_ext: bool = False):
        array = np.asarray(values, dtype=dtype).reshape(-1)
        bundle = self.constant_bundle({"value": array}, cache_key=("vector", _normalized_constant_name(str(name))))
        cur_limbs = int(self.context.L) - int(level)
        return bundle.plaintext(
            "value",
            state=fhe.CipherState(cur_limbs=cur_limbs, scale_degree=1,
                                  scaling_factor=self.context.scale_at(cur_limbs)),
            slots=self.max_slots if slots is None else int(slots),
            context=self.context,
            is_ext=bool(is_ext),
        )

    def constant_bundle(self, vectors: dict[str, np.ndarray], *, cache_key: object):
        arrays = {str(k): np.ascontiguousarray(v) for k, v in vectors.items()}
        source_bytes = sum(int(v.nbytes) for v in arrays.values())

        def factory(cache: bool):
            wrapped = {k: fhe.PackedRaw(torch.from_numpy(v)) for k, v in arrays.items()}
            return fhe.ConstantBundle(vectors=wrapped, cache_mode="plain" if cache else "none")

        if not self.plaintext_cache.accepts_source(source_bytes):
            return self.plaintext_cache.transient(factory, source_bytes=source_bytes)
        content = tuple((k, tuple(v.shape), v.dtype.str, _array_digest(v)) for k, v in sorted(arrays.items()))
        key = (_normalized_constant_name(cache_key), content)
        return self.plaintext_cache.get(key, factory, source_bytes=source_bytes)

    def plaintext_cache_info(self) -> dict[str, int]:
        return self.plaintext_cache.info()

    def clear_plaintext_cache(self) -> None:
        self.plaintext_cache.clear()

    def decrypt(self, cipher) -> np.ndarray:
        value = self.client.decrypt(cipher)
        return np.asarray(value).reshape(-1)


def plaintext_cache_snapshot(context) -> dict[str, int]:
    inspect = getattr(context, "plaintext_cache_info", None)
    if callable(inspect):
        return {k: int(v) for k, v in inspect().items()}
    return {k: 0 for k in ("entries", "bytes", "limit_bytes", "max_source_bytes", "hits", "misses", "skips")}


def release_if_supported(value) -> None:
    """Release explicit handles (ciphertexts, plaintexts, bundles) when the object has them."""

    release = getattr(value, "release", None)
    if callable(release):
        release()
        return
    constants = getattr(value, "constants", None)
    clear_cache = getattr(constants, "clear_cache", None)
    if callable(clear_cache):
        clear_cache()


def release_all(values) -> None:
    for value in values:
        release_if_supported(value)


def synchronize_device(device: str) -> None:
    torch.cuda.synchronize(torch.device(str(device)) if str(device).startswith("cuda") else None)


_STAGE_SYNC: bool | None = None


def stage_sync_enabled() -> bool:
    """True unless T2_STAGE_SYNC=0 (llama3fhe/backend.py:450-487)."""

    global _STAGE_SYNC
    if _STAGE_SYNC is None:
        _STAGE_SYNC = os.environ.get("T2_STAGE_SYNC", "1") != "0"
    return bool(_STAGE_SYNC)


def set_stage_sync(enabled: bool | None) -> None:
    global _STAGE_SYNC
    _STAGE_SYNC = None if enabled is None else bool(enabled)


def profile_sync_device(device: str) -> None:
    if stage_sync_enabled():
        synchronize_device(device)


def trim_device_allocator_cache(device: str) -> None:
    if os.environ.get("LLAMA_FHE_ALLOCATOR_TRIM", "") != "1" or not str(device).startswith("cuda"):
        return
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def cuda_memory_snapshot(device: str) -> dict[str, int | bool]:
    if not str(device).startswith("cuda") or not torch.cuda.is_available():
        return {"available": False}
    dev = torch.device(str(device))
    free_b, total_b = torch.cuda.mem_get_info(dev)
    return {
        "available": True,
        "allocator_allocated_bytes": int(torch.cuda.memory_allocated(dev)),
        "allocator_reserved_bytes": int(torch.cuda.memory_reserved(dev)),
        "allocator_peak_allocated_bytes": int(torch.cuda.max_memory_allocated(dev)),
        "allocator_peak_reserved_bytes": int(torch.cuda.max_memory_reserved(dev)),
        "device_used_bytes": int(total_b - free_b),
        "device_free_bytes": int(free_b),
        "device_total_bytes": int(total_b),
    }


def default_rotations(input_dim: int, block_out: int) -> set[int]:
    """Power-of-two rotation set of llama3fhe/backend.py:540-553."""

    input_dim, block_out = int(input_dim), int(block_out)
    if input_dim <= 0 or input_dim & (input_dim - 1):
        raise ValueError("input_dim must be a positive power of two.")
    if block_out <= 0 or block_out & (block_out - 1):
        raise ValueError("block_out must be a positive power of two.")
    rot = {block_out * (1 << i) for i in range(int(log2(input_dim)))}
    rot.update(1 << i for i in range(int(log2(block_out))))
    return rot


def create_sim_context(sim_cfg: SimulatorConfig, *, input_dim: int, block_out: int,
                       rotations=None, include_default_rotations: bool = True) -> EasyFHEContext:
    """Isolated-test context (llama3fhe/backend.py:556-596): keygen for the requested rotations."""

    requested = default_rotations(input_dim, block_out) if include_default_rotations else set()
    requested.update(int(v) for v in rotations or () if int(v))
    start = time.perf_counter()
    client, context = fhe.generate_client_context(
        fhe.CKKSContextSpec(
            depth=int(sim_cfg.maxLevelsRemaining),
            log_n=int(sim_cfg.logN),
            dnum=int(sim_cfg.dnum),
            dcrt_bits=int(sim_cfg.dcrtBits),
            first_mod=int(sim_cfg.firstMod),
            secret_key_dist=str(sim_cfg.secretKeyDist),
            scale_mode="fixed",
            rescale_policy=sim_cfg.rescale_policy(),
            rotations=tuple(sorted(requested)),
            auto_load_keys=True,
            scale_bits=int(sim_cfg.scaleBits),
        ),
        device=str(sim_cfg.device),
    )
    return EasyFHEContext(
        tensor=torch,
        fhe=fhe,
        client=client,
        context=context,
        max_slots=int(context.max_slots),
        keygen_wall_time_s=float(time.perf_counter() - start),
    )


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
