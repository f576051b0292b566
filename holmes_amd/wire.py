"""Ciphertext wire format.

The packet surface follows llama3fhe/parallel/wire.py (CipherMetadata, CipherPacket,
cipher_metadata, validate_cipher, rebuild_cipher, pack_cipher, unpack_cipher; lines 1-383): the
metadata records every component's full shape, dtype and device plus the state (cur_limbs,
scale_degree, scaling_factor) and the encoding contract (slots, batch_size, is_ext); packing stages
the components on the host as NumPy arrays (or keeps the device tensors by reference,
``host=False``); unpacking rebuilds on a device and refuses a packet whose metadata changed.

This backend adds one contiguous byte layout for a ciphertext, the same on the host and in HBM:

    header (64 bytes, little endian)
      0  magic b"HCKW"         4  version u16        6  flags u16 (1: is_ext, 2: checksum valid)
      8  components u16       10  limbs sent u16    12  log_n u8, 13 zero, 14 tag bytes u16
      16 batch u32            20  slots u32          24 scale_degree u32, 4 bytes zero
      32 scaling_factor f64   40  prime-chain fingerprint u64 (0: none)
      48 payload bytes u64    56  xxh64 of the payload (0 without flag 2)
    tag (utf-8, zero-padded to a multiple of 8 bytes)
    payload: component c, item b, limb l < limbs sent: N uint64 residues, in that order

Only the active limbs travel (a ciphertext at 9 of 24 stored limbs sends 9).  ``device_pack``
assembles the layout in one HBM buffer (one strided copy per component) so a batch of ciphertexts
crosses a link or PCIe as a single message; ``device_unpack`` rebuilds fresh component tensors
from it.  ``serialize`` / ``deserialize`` are the host forms with the payload checksum; the
prime-chain fingerprint makes a receiver with another context refuse the bytes.
"""

from __future__ import annotations

import copy
import hashlib
import struct
from dataclasses import dataclass
from typing import Iterable

import numpy as np
import torch

__all__ = [
    "CipherMetadata",
    "CipherPacket",
    "WireError",
    "cipher_metadata",
    "chain_fingerprint",
    "device_pack",
    "device_unpack",
    "deserialize",
    "pack_cipher",
    "rebuild_cipher",
    "serialize",
    "unpack_cipher",
    "validate_cipher",
    "wire_tag",
]

_ELEMENT_BYTES = {"uint64": 8, "int64": 8, "float64": 8, "complex128": 16, "uint32": 4, "int32": 4,
                  "float32": 4, "complex64": 8, "uint16": 2, "int16": 2, "float16": 2, "bfloat16": 2,
                  "uint8": 1, "int8": 1, "bool": 1}


class WireError(ValueError):
    """Malformed, corrupted or incompatible wire bytes."""


# ---------------------------------------------------------------------------- metadata / packets
def _components(cipher) -> tuple:
    cv = getattr(cipher, "cv", None)
    if cv is None:
        raise TypeError("cipher must expose a non-empty cv component sequence")
    if hasattr(cv, "dim"):
        cv = (cv,)
    try:
        cv = tuple(cv)
    except TypeError as exc:
        raise TypeError("cipher.cv must be iterable") from exc
    if not cv:
        raise ValueError("cipher.cv must not be empty")
    return cv


def _shape(x) -> tuple:
    s = getattr(x, "shape", None)
    if s is None:
        return ()
    try:
        return tuple(int(e) for e in s)
    except (TypeError, ValueError) as exc:
        raise TypeError(f"cipher component has invalid shape {s!r}") from exc


@dataclass(frozen=True)
class CipherMetadata:
    """Everything but the residues; shapes include the allocated limb capacity."""

    component_shapes: tuple
    component_dtypes: tuple
    component_devices: tuple
    cur_limbs: int
    scale_degree: int
    scaling_factor: float | None
    slots: int
    batch_size: int
    is_ext: bool

    @property
    def component_count(self) -> int:
        return len(self.component_shapes)

    @property
    def device(self) -> str | None:
        devs = {d for d in self.component_devices if d is not None}
        return next(iter(devs)) if len(devs) == 1 else None

    @property
    def nbytes(self) -> int:
        total = 0
        for shape, dtype in zip(self.component_shapes, self.component_dtypes):
            if dtype is None:
                continue
            eb = _ELEMENT_BYTES.get(str(dtype).removeprefix("torch."))
            if eb is not None:
                total += int(np.prod(shape, dtype=np.int64)) * eb if shape else eb
        return int(total)

    def without_devices(self) -> tuple:
        return (self.component_shapes, self.component_dtypes, self.cur_limbs, self.scale_degree,
                self.scaling_factor, self.slots, self.batch_size, self.is_ext)


def cipher_metadata(cipher) -> CipherMetadata:
    cv = _components(cipher)
    state = getattr(cipher, "state", None)
    if state is None:
        raise TypeError("cipher must expose state metadata")
    try:
        cur, deg = int(state.cur_limbs), int(state.scale_degree)
    except (AttributeError, TypeError, ValueError) as exc:
        raise TypeError("cipher.state must expose integer limb/scale fields") from exc
    if cur <= 0 or deg <= 0:
        raise ValueError(f"cipher state must be positive, got cur_limbs={cur}, scale_degree={deg}")
    sf = getattr(state, "scaling_factor", None)
    slots = int(getattr(cipher, "slots"))
    batch = int(getattr(cipher, "batch_size", 1))
    if slots <= 0 or batch <= 0:
        raise ValueError(f"slots/batch_size must be positive, got {slots}/{batch}")
    return CipherMetadata(
        component_shapes=tuple(_shape(c) for c in cv),
        component_dtypes=tuple(None if getattr(c, "dtype", None) is None else str(c.dtype) for c in cv),
        component_devices=tuple(None if getattr(c, "device", None) is None or not str(c.device) else str(c.device)
                                for c in cv),
        cur_limbs=cur, scale_degree=deg, scaling_factor=None if sf is None else float(sf), slots=slots,
        batch_size=batch, is_ext=bool(getattr(cipher, "is_ext", False)))


def validate_cipher(cipher, *, expected_device: str | None = None) -> CipherMetadata:
    md = cipher_metadata(cipher)
    devs = {d for d in md.component_devices if d is not None}
    if len(devs) > 1:
        raise ValueError(f"cipher components span multiple devices: {sorted(devs)}")
    if expected_device is not None and md.device is not None:
        want, got = str(expected_device), md.device
        if not (got == want or (want == "cuda" and got.startswith("cuda")) or (got == "cuda" and want.startswith("cuda"))):
            raise ValueError(f"cipher device {got!r} does not match {want!r}")
    for shape in md.component_shapes:
        if shape and md.batch_size != shape[0]:
            raise ValueError(f"cipher batch_size does not match component shape: {md.batch_size} vs {shape[0]}")
        if len(shape) >= 2 and md.cur_limbs > shape[-2]:
            raise ValueError(f"cipher cur_limbs={md.cur_limbs} exceeds component capacity {shape[-2]}")
    return md


def rebuild_cipher(template, components: Iterable):
    """``template``'s state and encoding around ``components`` (template unchanged)."""

    components = list(components)
    like = getattr(template, "cipher_like", None)
    if callable(like):
        return like(components)
    try:
        from .context import Cipher

        return Cipher(components, template.state, slots=int(template.slots), is_ext=bool(getattr(template, "is_ext", False)),
                      batch_size=int(getattr(template, "batch_size", 1)))
    except (AttributeError, TypeError, ValueError):  # a foreign cipher type without these fields
        clone = copy.copy(template)
        clone.cv = components
        return clone


def _to_host(c):
    if isinstance(c, np.ndarray):
        return np.array(c, copy=True)
    if callable(getattr(c, "numpy", None)):
        h = c.cpu() if callable(getattr(c, "cpu", None)) else c
        h = h.detach() if callable(getattr(h, "detach", None)) else h
        return np.array(h.numpy(), copy=True)
    return c.clone() if callable(getattr(c, "clone", None)) else c


def _to_device(c, device: str):
    if isinstance(c, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(c))
        return t.to(device) if str(device) != "cpu" else t.clone()
    to = getattr(c, "to", None)
    if callable(to):
        moved = to(str(device))
        if moved is c and callable(getattr(c, "clone", None)):
            moved = c.clone()
        return moved
    return c


@dataclass
class CipherPacket:
    """A ciphertext staged for a transport: metadata, components, a routing tag, the state."""

    metadata: CipherMetadata
    components: tuple
    tag: str = ""
    state: object | None = None

    @property
    def nbytes(self) -> int:
        return self.metadata.nbytes

    def validate(self) -> None:
        if len(self.components) != self.metadata.component_count:
            raise ValueError("packet component count does not match metadata")
        for c, shape in zip(self.components, self.metadata.component_shapes):
            if _shape(c) != shape:
                raise ValueError("packet component shape does not match metadata")


def pack_cipher(cipher, *, tag: str = "", host: bool = True) -> CipherPacket:
    """Metadata + components (host NumPy copies, or the device tensors by reference with
    ``host=False``); ``cipher`` is not consumed."""

    md = validate_cipher(cipher)
    comps = tuple(_to_host(c) for c in _components(cipher)) if host else tuple(_components(cipher))
    pkt = CipherPacket(metadata=md, components=comps, tag=str(tag), state=getattr(cipher, "state", None))
    pkt.validate()
    return pkt


class _Template:
    def __init__(self, pkt: CipherPacket):
        self.state = pkt.state
        self.slots = int(pkt.metadata.slots)
        self.is_ext = bool(pkt.metadata.is_ext)
        self.batch_size = int(pkt.metadata.batch_size)
        self.cv: list = []


def unpack_cipher(packet: CipherPacket, *, device: str = "cuda", template=None):
    """The cipher rebuilt on ``device`` (components never alias the sender's); refuses a packet
    whose metadata does not survive the trip."""

    packet.validate()
    comps = tuple(_to_device(c, str(device)) for c in packet.components)
    if template is None and packet.state is None:
        raise ValueError("packet has no state; pass a template cipher")
    out = rebuild_cipher(template if template is not None else _Template(packet), comps)
    after = validate_cipher(out, expected_device=str(device))
    if after.without_devices() != packet.metadata.without_devices():
        raise RuntimeError(f"cipher metadata changed during transport: sent={packet.metadata.without_devices()!r} "
                           f"got={after.without_devices()!r}")
    return out


# ---------------------------------------------------------------------------- binary layout
_MAGIC = b"HCKW"
_VERSION = 1
_HDR = struct.Struct("<4sHHHHB3xIII4xdQQQ")  # 64 bytes
assert _HDR.size == 64
_F_EXT, _F_SUM = 1, 2


def chain_fingerprint(primes) -> int:
    """64-bit fingerprint of a prime chain (blake2b of the primes as little-endian u64)."""

    data = np.asarray([int(p) for p in primes], dtype="<u8").tobytes()
    return int.from_bytes(hashlib.blake2b(data, digest_size=8).digest(), "little")


def _checksum(payload) -> int:
    import xxhash

    return xxhash.xxh64_intdigest(payload)


def _tag_bytes(tag: str) -> bytes:
    t = str(tag).encode("utf-8")
    if len(t) > 0xFFFF:
        raise ValueError("tag too long")
    return t + b"\0" * (-len(t) % 8)


def _header(md: CipherMetadata, log_n: int, fingerprint: int, payload_bytes: int, checksum: int | None, tag: bytes,
            tag_len: int) -> bytes:
    if md.scaling_factor is None:
        raise ValueError("the wire format needs a scaling factor")
    flags = (_F_EXT if md.is_ext else 0) | (_F_SUM if checksum is not None else 0)
    h = _HDR.pack(_MAGIC, _VERSION, flags, md.component_count, md.cur_limbs, int(log_n), md.batch_size, md.slots,
                  md.scale_degree, md.scaling_factor, int(fingerprint), int(payload_bytes), int(checksum or 0))
    # the tag length rides in bytes 14-15 (unused by the struct's padding after log_n)
    return h[:13] + b"\0" + struct.pack("<H", tag_len) + h[16:] + tag


def _parse(buf: bytes) -> dict:
    if len(buf) < _HDR.size:
        raise WireError("buffer shorter than the wire header")
    magic, ver, flags, comps, rows, log_n, batch, slots, deg, sf, fp, nbytes, chk = _HDR.unpack(
        bytes(buf[:_HDR.size]))
    if magic != _MAGIC:
        raise WireError("not a ciphertext wire buffer (bad magic)")
    if ver != _VERSION:
        raise WireError(f"unsupported wire version {ver}")
    tag_len = struct.unpack("<H", bytes(buf[14:16]))[0]
    n = 1 << log_n
    if nbytes != comps * batch * rows * n * 8:
        raise WireError("payload size does not match the header")
    return dict(flags=flags, comps=comps, rows=rows, n=n, batch=batch, slots=slots, deg=deg, sf=sf, fp=fp,
                nbytes=nbytes, chk=chk, tag_len=tag_len, tag_pad=tag_len + (-tag_len % 8))


def _active(cipher):
    """(metadata, the active-limb views of the components, limbs sent)."""

    md = validate_cipher(cipher)
    rows = md.cur_limbs if not md.is_ext else int(md.component_shapes[0][-2])
    return md, [c[:, :rows] for c in _components(cipher)], rows


def serialize(cipher, *, tag: str = "", primes=None, log_n: int | None = None, checksum: bool = True) -> bytes:
    """Host bytes of ``cipher`` (header, tag, active limbs, xxh64 of the payload)."""

    md, comps, rows = _active(cipher)
    n = int(comps[0].shape[-1])
    log_n = n.bit_length() - 1 if log_n is None else int(log_n)
    sizes = [int(c.numel()) * 8 for c in comps]
    tb = _tag_bytes(tag)
    lead = _HDR.size + len(tb)
    out = bytearray(lead + sum(sizes))
    words = np.frombuffer(out, dtype="<u8", offset=lead)
    pos = 0
    for c, k in zip(comps, sizes):
        src = c.view(torch.int64).cpu().numpy() if isinstance(c, torch.Tensor) else np.asarray(c)
        words[pos // 8:(pos + k) // 8] = src.reshape(-1).view(np.uint64)
        pos += k
    payload = memoryview(out)[lead:]
    fp = chain_fingerprint(primes) if primes is not None else 0
    head = _header(md, log_n, fp, len(payload), _checksum(payload) if checksum else None, tb,
                   len(str(tag).encode()))
    out[:lead] = head
    return bytes(out)


def _state_for(hdr, rows):
    from .context import CipherState

    return CipherState(cur_limbs=rows, scale_degree=hdr["deg"], scaling_factor=hdr["sf"])


def deserialize(buf, *, device: str = "cuda", primes=None):
    """The ciphertext of ``serialize``'s bytes on ``device`` (fresh tensors, exactly ``cur_limbs``
    limbs stored); checks magic, version, sizes, the checksum and, given ``primes``, the chain."""

    from .context import Cipher

    buf = memoryview(buf)
    h = _parse(buf)
    if primes is not None and h["fp"] and h["fp"] != chain_fingerprint(primes):
        raise WireError("the bytes were made under another prime chain")
    start = _HDR.size + h["tag_pad"]
    payload = buf[start:start + h["nbytes"]]
    if len(payload) != h["nbytes"]:
        raise WireError("truncated payload")
    if h["flags"] & _F_SUM and _checksum(payload) != h["chk"]:
        raise WireError("payload checksum mismatch")
    arr = np.frombuffer(payload, dtype="<u8").reshape(h["comps"], h["batch"], h["rows"], h["n"])
    cv = [_to_device(np.array(arr[c]), device) for c in range(h["comps"])]
    return Cipher(cv, _state_for(h, h["rows"]), slots=h["slots"], is_ext=bool(h["flags"] & _F_EXT),
                  batch_size=h["batch"])


def wire_tag(buf) -> str:
    """The routing tag stored in wire bytes (host buffer or a uint8 tensor's first bytes)."""

    if isinstance(buf, torch.Tensor):
        buf = buf[:_HDR.size + 0x10000].cpu().numpy().tobytes()
    h = _parse(memoryview(buf))
    return bytes(buf[_HDR.size:_HDR.size + h["tag_len"]]).decode("utf-8")


def device_pack(ciphers, *, tags=None, primes=None, out: torch.Tensor | None = None) -> torch.Tensor:
    """One uint8 buffer on the ciphertexts' device holding every cipher's wire layout back to back
    (no checksum: a device-to-device or pinned transfer), built by one strided copy per component.
    ``out`` (a large enough uint8 tensor) is reused when given."""

    ciphers = [ciphers] if not isinstance(ciphers, (list, tuple)) else list(ciphers)
    tags = [""] * len(ciphers) if tags is None else [str(t) for t in tags]
    fp = chain_fingerprint(primes) if primes is not None else 0
    parts = []
    total = 0
    for ct, tag in zip(ciphers, tags):
        md, comps, rows = _active(ct)
        n = int(comps[0].shape[-1])
        nb = sum(int(c.numel()) for c in comps) * 8
        hdr = _header(md, n.bit_length() - 1, fp, nb, None, _tag_bytes(tag), len(tag.encode()))
        parts.append((hdr, comps, nb))
        total += len(hdr) + nb
    dev = ciphers[0].cv[0].device
    buf = out if out is not None else torch.empty(total, dtype=torch.uint8, device=dev)
    if buf.numel() < total or buf.dtype != torch.uint8:
        raise ValueError(f"out needs {total} uint8 bytes")
    blob = b"".join(h for h, _, _ in parts)
    staged = torch.empty(len(blob), dtype=torch.uint8, pin_memory=dev.type == "cuda")
    staged.numpy()[:] = np.frombuffer(blob, dtype=np.uint8)
    heads = staged.to(dev, non_blocking=True)  # one upload of every header
    pos = hpos = 0
    for hdr, comps, nb in parts:
        buf[pos:pos + len(hdr)].copy_(heads[hpos:hpos + len(hdr)])
        pos += len(hdr)
        hpos += len(hdr)
        for c in comps:
            k = int(c.numel()) * 8
            # int64 views: torch's vectorised copy (its uint64 copies take a slow generic path)
            buf[pos:pos + k].view(torch.int64).view(c.shape).copy_(c.view(torch.int64))
            pos += k
    return buf[:total]


def device_unpack(buf: torch.Tensor, *, primes=None, count: int | None = None) -> list:
    """The ciphertexts of a ``device_pack`` buffer, as fresh tensors on the buffer's device."""

    from .context import Cipher

    out = []
    pos = 0
    total = int(buf.numel())
    while pos < total and (count is None or len(out) < count):
        head = buf[pos:pos + _HDR.size].cpu().numpy().tobytes()
        h = _parse(memoryview(head))
        if primes is not None and h["fp"] and h["fp"] != chain_fingerprint(primes):
            raise WireError("the bytes were made under another prime chain")
        pos += _HDR.size + h["tag_pad"]
        if pos + h["nbytes"] > total:
            raise WireError("truncated payload")
        shape = (h["batch"], h["rows"], h["n"])
        step = h["batch"] * h["rows"] * h["n"] * 8
        cv = []
        for _ in range(h["comps"]):
            cv.append(buf[pos:pos + step].view(torch.int64).view(shape).clone().view(torch.uint64))
            pos += step
        out.append(Cipher(cv, _state_for(h, h["rows"]), slots=h["slots"], is_ext=bool(h["flags"] & _F_EXT),
                          batch_size=h["batch"]))
    return out
