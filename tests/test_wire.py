"""CPU tests of the ciphertext wire format: the packet protocol of llama3fhe/parallel/wire.py
(metadata, host staging, rebuild without aliasing, pickling, validation; the behaviours of the
reference's tests/test_parallel_wire.py) and this backend's byte layout (host and buffer forms:
round trips with only the active limbs, tags, the checksum, the chain fingerprint, malformed
input), on CPU tensors."""

from __future__ import annotations

import pickle
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from holmes_amd import wire
from holmes_amd.context import Cipher, CipherState

N = 16


def _cipher(batch=1, rows=5, limbs=3, seed=0, comps=2, is_ext=False):
    rng = np.random.default_rng(seed)
    cv = [torch.from_numpy(rng.integers(0, 2**50, (batch, rows, N), dtype=np.uint64)) for _ in range(comps)]
    return Cipher(cv, CipherState(cur_limbs=limbs, scale_degree=1, scaling_factor=2.0**40), slots=N // 2,
                  is_ext=is_ext, batch_size=batch)


def test_metadata_and_size():
    md = wire.cipher_metadata(_cipher())
    assert md.component_count == 2 and md.cur_limbs == 3 and md.scaling_factor == 2.0**40
    assert md.device == "cpu" and md.nbytes == 2 * 5 * N * 8 and md.slots == N // 2


def test_host_packet_round_trip_and_pickle():
    ct = _cipher(seed=1)
    pkt = wire.pack_cipher(ct, tag="attn_in/lane/3")
    assert pkt.tag == "attn_in/lane/3" and all(isinstance(c, np.ndarray) for c in pkt.components)
    clone = pickle.loads(pickle.dumps(pkt))
    back = wire.unpack_cipher(clone, device="cpu", template=ct)
    for a, b in zip(back.cv, ct.cv):
        assert torch.equal(a, b) and a.data_ptr() != b.data_ptr()
    no_template = wire.unpack_cipher(pkt, device="cpu")
    assert no_template.state.cur_limbs == 3 and no_template.slots == N // 2
    pkt.state = None
    with pytest.raises(ValueError):
        wire.unpack_cipher(pkt, device="cpu")


def test_packet_by_reference_and_metadata_check():
    ct = _cipher(seed=2)
    pkt = wire.pack_cipher(ct, host=False)
    assert pkt.components[0] is ct.cv[0]
    out = wire.unpack_cipher(pkt, device="cpu", template=ct)
    assert out.cv[0] is not ct.cv[0] and torch.equal(out.cv[0], ct.cv[0])
    bad = wire.pack_cipher(ct)
    bad.components = (bad.components[0][:, :4],) + bad.components[1:]
    with pytest.raises(ValueError, match="shape"):
        wire.unpack_cipher(bad, device="cpu", template=ct)


def test_validation_rejects_bad_ciphers():
    ct = _cipher()
    ct.state = ct.state.replace(cur_limbs=6)
    with pytest.raises(ValueError, match="capacity"):
        wire.validate_cipher(ct)
    fake = SimpleNamespace(cv=[SimpleNamespace(shape=(2, 4, 8), dtype="torch.uint64", device="cuda:0"),
                               SimpleNamespace(shape=(2, 4, 8), dtype="torch.uint64", device="cuda:1")],
                           state=SimpleNamespace(cur_limbs=2, scale_degree=1, scaling_factor=1.0), slots=4,
                           batch_size=2)
    with pytest.raises(ValueError, match="multiple devices"):
        wire.validate_cipher(fake)
    fake.cv[1].device = "cuda:0"
    fake.batch_size = 3
    with pytest.raises(ValueError, match="batch_size"):
        wire.validate_cipher(fake)
    with pytest.raises(ValueError, match="does not match"):
        wire.validate_cipher(_cipher(), expected_device="cuda")


@pytest.mark.parametrize("batch,rows,limbs", [(1, 5, 3), (3, 7, 7), (2, 4, 1)])
def test_bytes_round_trip_sends_only_active_limbs(batch, rows, limbs):
    ct = _cipher(batch, rows, limbs, seed=batch + rows)
    primes = [97, 193, 257]
    buf = wire.serialize(ct, tag="pairfm/partial/2", primes=primes)
    assert len(buf) == 64 + 16 + 2 * batch * limbs * N * 8
    assert wire.wire_tag(buf) == "pairfm/partial/2"
    back = wire.deserialize(buf, device="cpu", primes=primes)
    assert back.state.cur_limbs == limbs and back.batch_size == batch and back.slots == N // 2
    assert back.state.scaling_factor == 2.0**40 and not back.is_ext
    for a, b in zip(back.cv, ct.cv):
        assert a.shape == (batch, limbs, N) and torch.equal(a, b[:, :limbs])


def test_bytes_detect_corruption_and_foreign_chains():
    ct = _cipher(seed=5)
    buf = bytearray(wire.serialize(ct, primes=[97, 193]))
    flipped = bytearray(buf)
    flipped[-3] ^= 0x10
    with pytest.raises(wire.WireError, match="checksum"):
        wire.deserialize(bytes(flipped), device="cpu")
    with pytest.raises(wire.WireError, match="prime chain"):
        wire.deserialize(bytes(buf), device="cpu", primes=[97, 257])
    with pytest.raises(wire.WireError, match="magic"):
        wire.deserialize(b"XXXX" + bytes(buf[4:]), device="cpu")
    with pytest.raises(wire.WireError, match="version"):
        wire.deserialize(bytes(buf[:4]) + b"\x07\x00" + bytes(buf[6:]), device="cpu")
    with pytest.raises(wire.WireError, match="truncated"):
        wire.deserialize(bytes(buf[:-8]), device="cpu")
    with pytest.raises(wire.WireError):
        wire.deserialize(bytes(buf[:40]), device="cpu")
    unchecked = wire.serialize(ct, checksum=False)
    raw = bytearray(unchecked)
    raw[-3] ^= 0x10
    assert not torch.equal(wire.deserialize(bytes(raw), device="cpu").cv[1], ct.cv[1][:, :3])


def test_buffer_form_holds_several_ciphertexts():
    cts = [_cipher(1, 5, 3, seed=7), _cipher(2, 6, 6, seed=8), _cipher(1, 9, 9, seed=9, is_ext=True)]
    buf = wire.device_pack(cts, tags=["a", "bb", "extended"], primes=[97])
    assert buf.dtype == torch.uint8 and buf.device.type == "cpu"
    back = wire.device_unpack(buf, primes=[97])
    assert len(back) == 3 and back[2].is_ext
    for got, want in zip(back, cts):
        rows = got.state.cur_limbs if not want.is_ext else want.cv[0].shape[1]
        for a, b in zip(got.cv, want.cv):
            assert torch.equal(a, b[:, :rows])
    assert wire.wire_tag(buf) == "a"
    with pytest.raises(wire.WireError):
        wire.device_unpack(buf, primes=[101])
    # the buffer form is the byte form without the checksum
    one = wire.device_pack(cts[0])
    assert wire.deserialize(one.numpy().tobytes(), device="cpu").state.cur_limbs == 3
    out = torch.empty(one.numel() + 64, dtype=torch.uint8)
    assert torch.equal(wire.device_pack(cts[0], out=out), one)


@pytest.mark.parametrize("form", ["bytes", "buffer"])
def test_extended_basis_ciphers_keep_rows_and_limbs_apart(form):
    """An extended-basis ciphertext stores cur_limbs Q limbs plus the special-prime limbs: all of its
    rows travel, and the receiver gets cur_limbs back from the header, not the row count."""
    ct = _cipher(batch=2, rows=5, limbs=3, seed=11, is_ext=True)  # 3 Q limbs + 2 special limbs
    if form == "bytes":
        buf = wire.serialize(ct, primes=[97, 193])
        assert len(buf) == 64 + 2 * 2 * 5 * N * 8
        back = wire.deserialize(buf, device="cpu", primes=[97, 193])
    else:
        (back,) = wire.device_unpack(wire.device_pack(ct, primes=[97, 193]), primes=[97, 193])
    assert back.is_ext and back.state.cur_limbs == 3 and back.batch_size == 2
    for a, b in zip(back.cv, ct.cv):
        assert a.shape == (2, 5, N) and torch.equal(a, b)


def test_header_rejects_more_limbs_than_rows():
    buf = bytearray(wire.serialize(_cipher(rows=5, limbs=3, seed=12)))
    buf[12:14] = (4).to_bytes(2, "little")  # cur_limbs 4 > the 3 rows sent
    with pytest.raises(wire.WireError, match="rows"):
        wire.deserialize(bytes(buf), device="cpu")
