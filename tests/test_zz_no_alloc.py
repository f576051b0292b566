"""hck_rotate_noalloc (the rotation entry point that allocates nothing: its key-switch workspace is
a fixed device array inside the library) against hck_rotate, both through the C ABI: bit-identical
outputs on two calls in a row, the second smaller than the first (fewer limbs, one item, the
accumulating form), a batch that runs as several launches through the array, and a level whose
one-item workspace exceeds the array refused before anything is launched."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

N = 1 << 16


@pytest.fixture(scope="module")
def env():
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=23, dnum=3, seed=20261207, rotations=(1, 3))
    client, ctx = fhe.generate_client_context(spec, device="cuda")
    return ctx


def _rand(ctx, rng, batch, limbs):
    q = np.array(ctx.primes[:limbs], dtype=np.uint64).reshape(1, limbs, 1)
    return torch.from_numpy(rng.integers(0, 1 << 62, size=(batch, limbs, N), dtype=np.uint64) % q).cuda()


def _both(ctx, limbs, batch, rotation, acc):
    """(hck_rotate outputs, hck_rotate_noalloc outputs) for one random input."""

    from holmes_amd import _native as nat

    L = nat.lib()
    rng = np.random.default_rng(limbs * 100 + batch)
    c0, c1 = _rand(ctx, rng, batch, limbs), _rand(ctx, rng, batch, limbs)
    g = ctx.galois_element(rotation)
    keys = nat.ptr_array([ctx.key_for_galois(g).data_ptr()] * batch)
    a0 = _rand(ctx, rng, batch, limbs) if acc else None
    a1 = _rand(ctx, rng, batch, limbs) if acc else None
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for noalloc in (False, True):
        o0, o1 = ctx.empty(batch, limbs, N), ctx.empty(batch, limbs, N)
        args = [ctx.handle, limbs, batch, g, c0.data_ptr(), c1.data_ptr(), limbs * N, keys,
                a0.data_ptr() if acc else None, a1.data_ptr() if acc else None, limbs * N if acc else 0,
                o0.data_ptr(), o1.data_ptr(), limbs * N]
        if noalloc:
            rc = L.hck_rotate_noalloc(*args, stream)
        else:
            ws = ctx.workspace(L.hck_rotate_workspace_bytes(ctx.handle, limbs, batch))
            rc = L.hck_rotate(*args, ws.data_ptr(), ws.numel(), stream)
        assert rc == 0, (noalloc, rc)
        outs.append((o0, o1))
    torch.cuda.synchronize()
    return outs


def test_noalloc_rotation_matches_hck_rotate_twice(env):
    ctx = env
    print("no-alloc rotation: call 1 (2 items, 24 limbs: two one-item launches), call 2 (1 item, 5 limbs, "
          "accumulating)", flush=True)
    for limbs, batch, rotation, acc in ((24, 2, 1, False), (5, 1, 3, True)):
        (w0, w1), (g0, g1) = _both(ctx, limbs, batch, rotation, acc)
        assert torch.equal(w0.view(torch.int64), g0.view(torch.int64)), (limbs, batch)
        assert torch.equal(w1.view(torch.int64), g1.view(torch.int64)), (limbs, batch)


def test_noalloc_batches_beyond_one_launch(env):
    """At 12 limbs 5 items of key-switch workspace exceed the array, so they run as several launches
    through it, and still equal hck_rotate bit for bit."""

    from holmes_amd import _native as nat

    ctx = env
    L = nat.lib()
    assert L.hck_rotate_noalloc_limit(ctx.handle, 12) == 1 << 30
    assert L.hck_rotate_workspace_bytes(ctx.handle, 12, 5) > nat.HCK_NOALLOC_SCRATCH_BYTES
    (w0, w1), (g0, g1) = _both(ctx, 12, 5, 3, True)
    assert torch.equal(w0.view(torch.int64), g0.view(torch.int64))
    assert torch.equal(w1.view(torch.int64), g1.view(torch.int64))


def test_noalloc_rejects_levels_beyond_its_array():
    """At 38 limbs with dnum 5 one item's key-switch workspace (322 limbs, 161 MiB) exceeds the
    128 MiB array: the call is refused before anything is launched, and the limit says 0."""

    from holmes_amd import _native as nat
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=37, dnum=5, dcrt_bits=50, first_mod=50, scale_bits=50, seed=20261208)
    _, ctx = fhe.generate_client_context(spec, device="cuda")
    L = nat.lib()
    assert L.hck_rotate_workspace_bytes(ctx.handle, 38, 1) > nat.HCK_NOALLOC_SCRATCH_BYTES
    assert L.hck_rotate_noalloc_limit(ctx.handle, 38) == 0
    assert L.hck_rotate_noalloc_limit(ctx.handle, 24) == 1 << 30
    x = ctx.empty(2, 38, N)
    out = ctx.empty(2, 38, N)
    g = ctx.galois_element(1)
    key = torch.zeros(8, dtype=torch.uint64, device="cuda")  # never read: the call is refused first
    keys = nat.ptr_array([key.data_ptr()])
    rc = L.hck_rotate_noalloc(ctx.handle, 38, 1, g, x[0].data_ptr(), x[1].data_ptr(), 38 * N, keys, None, None,
                              0, out[0].data_ptr(), out[1].data_ptr(), 38 * N, torch.cuda.current_stream().cuda_stream)
    assert rc == nat.HCK_ERR_SCRATCH
    assert b"scratch" in L.hck_error_string(rc)
