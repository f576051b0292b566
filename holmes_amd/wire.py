"""Ciphertext wire format.

The packet surface keeps the names and contract of llama3fhe/parallel/wire.py (CipherMetadata,
CipherPacket, cipher_metadata, validate_cipher, rebuild_cipher, pack_cipher, unpack_cipher;
lines 1-383): metadata = every component's full shape, dtype and device, the state (cur_limbs,
scale_degree, scaling_factor) and the encoding (slots, batch_size, is_ext); a packet holds host
NumPy copies (or, ``host=False``, the device tensors themselves); unpacking places fresh tensors
on a device and refuses a result whose metadata differs from what was sent.

This backend adds one contiguous byte layout for a ciphertext, the same on the host and in HBM:

    header (64 bytes, little endian)
      0  magic b"HCKW"         4  version u16 (2)    6  flags u16 (1: is_ext, 2: checksum valid)
      8  components u16       10  rows sent u16     12  cur_limbs u16     14 tag bytes u16
      16 batch u32            20  slots u32          24 scale_degree u32   28 log_n u8, 3 zero
      32 scaling_factor f64   40  prime-chain fingerprint u64 (0: none)
      48 payload bytes u64    56  xxh64 of the payload (0 without flag 2)
    tag (utf-8, zero-padded to a multiple of 8 bytes)
    payload: component c, item b, row r < rows sent: N uint64 residues, in that order

Only the active rows travel: cur_limbs rows of a ciphertext in the Q basis (a ciphertext at 9 of
24 stored limbs sends 9), every stored row (cur_limbs Q limbs + the special-prime limbs) of an
extended-basis one; the header keeps the row count and cur_limbs apart.  ``device_pack``
assembles the layout in one HBM buffer (one strided copy per component) so a batch of ciphertexts
crosses a link or PCIe as a single message; ``device_unpack`` rebuilds fresh component tensors
from it.  ``serialize`` / ``deserialize`` are the host forms with the payload checksum; the
prime-chain fingerprint makes a receiver with another context refuse the bytes.
"""

from __future__ import annotations

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

class WireError(ValueError):
    """Malformed, corrupted or incompatible wire bytes."""


# ---------------------------------------------------------------------------- metadata / packets
def _itemsize(dtype) -> int | None:
    """Bytes per element of a torch or NumPy dtype (or its string form), None if unknown."""

    if dtype is None:
        return None
    name = str(dtype).rsplit(".", 1)[-1]
    tdt = getattr(torch, name, None)
    if isinstance(tdt, torch.dtype):
        return int(tdt.itemsize)
    try:
        return int(np.dtype(name).itemsize)
    except TypeError:
        return None


def _describe(component) -> tuple:
    """(shape, dtype string or None, device string or None) of one component."""

    shape = getattr(component, "shape", None)
    try:
        shape = () if shape is None else tuple(int(d) for d in shape)
    except (TypeError, ValueError) as exc:
        raise TypeError(f"a ciphertext component reports an unusable shape {shape!r}") from exc
    dtype = getattr(component, "dtype", None)
    device = getattr(component, "device", None)
    return shape, None if dtype is None else str(dtype), (str(device) or None) if device is not None else None


def _component_list(cipher) -> tuple:
    cv = getattr(cipher, "cv", None)
    if cv is None:
        raise TypeError(f"{type(cipher).__name__} has no cv component list")
    items = (cv,) if hasattr(cv, "dim") else tuple(cv) if isinstance(cv, (list, tuple)) else None
    if items is None:
        raise TypeError("cipher.cv is neither a tensor nor a list / tuple of components")
    if not items:
        raise ValueError("cipher.cv holds no component")
    return items


@dataclass(frozen=True)
class CipherMetadata:
    """A ciphertext without its residues: per-component shape (allocated limb capacity included),
    dtype and device; the state (cur_limbs, scale_degree, scaling_factor); slots, batch, basis."""

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
        named = set(filter(None, self.component_devices))
        return named.pop() if len(named) == 1 else None

    @property
    def nbytes(self) -> int:
        total = 0
        for shape, dtype in zip(self.component_shapes, self.component_dtypes):
            size = _itemsize(dtype)
            if size:
                total += size * int(np.prod(shape, dtype=np.int64))
        return total

    def without_devices(self) -> tuple:
        """Everything a transport must preserve (the device may legitimately change)."""

        return (self.component_shapes, self.component_dtypes, self.cur_limbs, self.scale_degree,
                self.scaling_factor, self.slots, self.batch_size, self.is_ext)


def cipher_metadata(cipher) -> CipherMetadata:
    comps = _component_list(cipher)
    state = getattr(cipher, "state", None)
    try:
        limbs, degree = int(state.cur_limbs), int(state.scale_degree)
    except (AttributeError, TypeError, ValueError) as exc:
        raise TypeError("cipher.state needs integer cur_limbs and scale_degree") from exc
    slots, batch = int(getattr(cipher, "slots")), int(getattr(cipher, "batch_size", 1))
    if min(limbs, degree, slots, batch) < 1:
        raise ValueError(f"cur_limbs {limbs}, scale_degree {degree}, slots {slots} and batch_size {batch} "
                         "must all be positive")
    scale = getattr(state, "scaling_factor", None)
    shapes, dtypes, devices = zip(*map(_describe, comps))
    return CipherMetadata(component_shapes=tuple(shapes), component_dtypes=tuple(dtypes),
                          component_devices=tuple(devices), cur_limbs=limbs, scale_degree=degree,
                          scaling_factor=None if scale is None else float(scale), slots=slots, batch_size=batch,
                          is_ext=bool(getattr(cipher, "is_ext", False)))


def _same_device(have: str, want: str) -> bool:
    """Equal device names, where a bare "cuda" matches any "cuda:<i>"."""

    if have == want:
        return True
    return "cuda" in (have, want) and have.startswith("cuda") and want.startswith("cuda")


def validate_cipher(cipher, *, expected_device: str | None = None) -> CipherMetadata:
    """Metadata of ``cipher`` after the checks a transport relies on: one device (``expected_device``
    when given), batch_size equal to every component's leading extent, cur_limbs within capacity."""

    md = cipher_metadata(cipher)
    named = sorted(set(filter(None, md.component_devices)))
    if len(named) > 1:
        raise ValueError(f"components live on multiple devices {named}; a packet needs one")
    if expected_device is not None and md.device is not None and not _same_device(md.device, str(expected_device)):
        raise ValueError(f"components are on {md.device!r}, which does not match {str(expected_device)!r}")
    for shape in md.component_shapes:
        if shape and shape[0] != md.batch_size:
            raise ValueError(f"batch_size {md.batch_size} disagrees with a component's leading extent {shape[0]}")
        if len(shape) > 1 and shape[-2] < md.cur_limbs:
            raise ValueError(f"cur_limbs {md.cur_limbs} is above the component's limb capacity {shape[-2]}")
    return md


def rebuild_cipher(template, components: Iterable):
    """A ciphertext around ``components`` with ``template``'s state and encoding.  A template with
    ``cipher_like`` (any ciphertext of this backend) builds it; otherwise the template only has to
    carry ``state``, ``slots``, ``is_ext`` and ``batch_size`` -- a packet's metadata does -- and a
    Cipher of this backend is made from them."""

    comps = list(components)
    if callable(getattr(template, "cipher_like", None)):
        return template.cipher_like(comps)
    from .context import Cipher

    missing = [k for k in ("state", "slots") if getattr(template, k, None) is None]
    if missing:
        raise TypeError(f"a rebuild template needs {', '.join(missing)} (or a cipher_like method)")
    return Cipher(comps, template.state, slots=int(template.slots), is_ext=bool(getattr(template, "is_ext", False)),
                  batch_size=int(getattr(template, "batch_size", 1)))


def _host_copy(component):
    """A host NumPy copy of a tensor (any device), or an independent copy of anything else."""

    if isinstance(component, torch.Tensor):
        return component.detach().cpu().numpy().copy()
    if isinstance(component, np.ndarray):
        return component.copy()
    return component.clone() if callable(getattr(component, "clone", None)) else component


def _placed(component, device: str):
    """``component`` as a tensor on ``device`` that shares no storage with the original."""

    if isinstance(component, np.ndarray):
        fresh = torch.from_numpy(np.ascontiguousarray(component).copy())
        return fresh if str(device) == "cpu" else fresh.to(device)
    if isinstance(component, torch.Tensor):
        moved = component.to(str(device))
        return moved.clone() if moved.data_ptr() == component.data_ptr() else moved
    return component


@dataclass
class CipherPacket:
    """A ciphertext staged for a transport: metadata, components, a routing tag and the state."""

    metadata: CipherMetadata
    components: tuple
    tag: str = ""
    state: object | None = None

    @property
    def nbytes(self) -> int:
        return self.metadata.nbytes

    def validate(self) -> None:
        want = self.metadata.component_shapes
        if len(self.components) != len(want):
            raise ValueError(f"packet carries {len(self.components)} components, metadata lists {len(want)}")
        got = tuple(_describe(c)[0] for c in self.components)
        if got != want:
            raise ValueError(f"packet component shape {got} does not match metadata {want}")


def pack_cipher(cipher, *, tag: str = "", host: bool = True) -> CipherPacket:
    """A packet of ``cipher`` (not consumed): host NumPy copies of the components, or with
    ``host=False`` the device tensors themselves."""

    md = validate_cipher(cipher)
    comps = _component_list(cipher)
    packet = CipherPacket(metadata=md, components=tuple(map(_host_copy, comps)) if host else comps, tag=str(tag),
                          state=getattr(cipher, "state", None))
    packet.validate()
    return packet


def unpack_cipher(packet: CipherPacket, *, device: str = "cuda", template=None):
    """The packet's ciphertext on ``device`` (its components never share storage with the sender's).
    Without a ``template`` the packet's own state is used.  A result whose metadata differs from
    the packet's (apart from the device) is refused."""

    packet.validate()
    if template is None and packet.state is None:
        raise ValueError("the packet carries no state; pass a template ciphertext")
    comps = [_placed(c, str(device)) for c in packet.components]
    if template is None:
        from types import SimpleNamespace

        md = packet.metadata
        template = SimpleNamespace(state=packet.state, slots=md.slots, is_ext=md.is_ext, batch_size=md.batch_size)
    result = rebuild_cipher(template, comps)
    arrived = validate_cipher(result, expected_device=str(device)).without_devices()
    sent = packet.metadata.without_devices()
    if arrived != sent:
        raise RuntimeError(f"the ciphertext arrived with other metadata than it was sent with: {sent!r} -> {arrived!r}")
    return result


# ---------------------------------------------------------------------------- binary layout
_MAGIC = b"HCKW"
_VERSION = 2
_HDR = struct.Struct("<4sHHHHHHIIIB3xdQQQ")  # 64 bytes
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


def _header(md: CipherMetadata, rows: int, log_n: int, fingerprint: int, payload_bytes: int, checksum: int | None,
            tag: bytes, tag_len: int) -> bytes:
    if md.scaling_factor is None:
        raise ValueError("the wire format needs a scaling factor")
    if max(rows, md.cur_limbs, md.component_count, tag_len) > 0xFFFF:
        raise ValueError("rows, cur_limbs, components and tag length must each fit 16 bits")
    flags = (_F_EXT if md.is_ext else 0) | (_F_SUM if checksum is not None else 0)
    return _HDR.pack(_MAGIC, _VERSION, flags, md.component_count, int(rows), md.cur_limbs, int(tag_len),
                     md.batch_size, md.slots, md.scale_degree, int(log_n), md.scaling_factor, int(fingerprint),
                     int(payload_bytes), int(checksum or 0)) + tag


def _parse(buf: bytes) -> dict:
    if len(buf) < _HDR.size:
        raise WireError("buffer shorter than the wire header")
    magic, ver, flags, comps, rows, limbs, tag_len, batch, slots, deg, log_n, sf, fp, nbytes, chk = _HDR.unpack(
        bytes(buf[:_HDR.size]))
    if magic != _MAGIC:
        raise WireError("not a ciphertext wire buffer (bad magic)")
    if ver != _VERSION:
        raise WireError(f"unsupported wire version {ver}")
    if not 0 < limbs <= rows or log_n > 20:
        raise WireError(f"header holds {rows} rows for {limbs} limbs at log N {log_n}")
    n = 1 << log_n
    if nbytes != comps * batch * rows * n * 8:
        raise WireError("payload size does not match the header")
    return dict(flags=flags, comps=comps, rows=rows, limbs=limbs, n=n, batch=batch, slots=slots, deg=deg, sf=sf,
                fp=fp, nbytes=nbytes, chk=chk, tag_len=tag_len, tag_pad=tag_len + (-tag_len % 8))


def _active(cipher):
    """(metadata, the views of the rows that travel, rows sent)."""

    md = validate_cipher(cipher)
    rows = md.cur_limbs if not md.is_ext else int(md.component_shapes[0][-2])
    return md, [c[:, :rows] for c in _component_list(cipher)], rows


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
    head = _header(md, rows, log_n, fp, len(payload), _checksum(payload) if checksum else None, tb,
                   len(str(tag).encode()))
    out[:lead] = head
    return bytes(out)


def _state_for(hdr):
    from .context import CipherState

    return CipherState(cur_limbs=hdr["limbs"], scale_degree=hdr["deg"], scaling_factor=hdr["sf"])


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
    cv = [_placed(arr[c], device) for c in range(h["comps"])]
    return Cipher(cv, _state_for(h), slots=h["slots"], is_ext=bool(h["flags"] & _F_EXT), batch_size=h["batch"])


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
        hdr = _header(md, rows, n.bit_length() - 1, fp, nb, None, _tag_bytes(tag), len(tag.encode()))
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
        out.append(Cipher(cv, _state_for(h), slots=h["slots"], is_ext=bool(h["flags"] & _F_EXT),
                          batch_size=h["batch"]))
    return out
