"""holmes_encode_stage2, the reference's encode sidecar entry point, bound through ctypes with the
argtypes the reference declares (bench/cmp/holmes_fast_stage2.py:37) and called the way it calls it
(:71-85): the context's QplusP_map / QmaxdiffplusPmaxdiff_map / QbarretRatioplusPbarretRatio_map /
QbarretKplusPbarretK_map rows for the limb count and its power_of_roots(_shoup) tables, as device
pointers.  The input is the oracle's special-IFFT output (the sidecar's stage-1 input, interleaved
Re / Im per slot); the residues must equal the oracle's whole encoder bit for bit, on the 50-bit
chain and on the reference's 60/59-bit chain (assets/feature_major.json), in one launch, in row
batches, and as the two kernels launched separately (parts 1 then 2)."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402

N = 1 << 16


def _bound():
    from holmes_amd import _native as nat

    lib = ctypes.CDLL(str(nat.LIB_PATH))
    p, i, ll, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_double
    lib.holmes_encode_stage2.argtypes = [p, p, ll, i, d, i, p, p, p, p, p, p, p, i, i, i]
    lib.holmes_encode_stage2.restype = i
    return lib


def _context(chain):
    from holmes_amd import fhe

    if chain == "50":
        spec = fhe.CKKSContextSpec(depth=7, dnum=2, dcrt_bits=50, first_mod=50, scale_bits=40, seed=20261240)
    else:
        spec = fhe.CKKSContextSpec(depth=7, dnum=2, dcrt_bits=59, first_mod=60, scale_bits=59, seed=20261241)
    _, ctx = fhe.generate_client_context(spec, device="cuda")
    return ctx


def _stage2(lib, ctx, w, scale, limbs, rows_per_launch=0, parts=3, out=None):
    rows = w.shape[0]
    win = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    if out is None:
        out = torch.zeros((rows, limbs, N), dtype=torch.uint64, device="cuda")
    rc = lib.holmes_encode_stage2(
        out.data_ptr(), win.data_ptr(), int(win.stride(0)), rows, float(scale), limbs,
        ctx.QplusP_map[limbs].data_ptr(), ctx.QmaxdiffplusPmaxdiff_map[limbs].data_ptr(),
        ctx.QbarretRatioplusPbarretRatio_map[limbs].data_ptr(), ctx.QbarretKplusPbarretK_map[limbs].data_ptr(),
        ctx.power_of_roots.data_ptr(), ctx.power_of_roots_shoup.data_ptr(),
        torch.cuda.current_stream().cuda_stream, rows_per_launch, parts, 0)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("chain", ["50", "60/59"])
def test_encode_stage2_matches_oracle_encoder(chain):
    ctx = _context(chain)
    lib = _bound()
    limbs = 5
    scale = 2.0**40 if chain == "50" else 2.0**55
    print(f"holmes_encode_stage2: chain {chain}, {limbs} limbs, scale 2^{np.log2(scale):.0f}", flush=True)
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    rng = np.random.default_rng(91)
    rows = 3
    values = rng.uniform(-4, 4, size=(rows, N // 2))
    w = np.stack([orc.encode_stage1(v) for v in values])
    want = np.stack([orc.encode_real(v, scale, list(range(limbs)))[0] for v in values])
    got = _stage2(lib, ctx, w, scale, limbs).cpu().numpy()
    assert np.array_equal(got, want)
    batched = _stage2(lib, ctx, w, scale, limbs, rows_per_launch=2).cpu().numpy()
    assert np.array_equal(batched, want)
    two = _stage2(lib, ctx, w, scale, limbs, parts=1)
    two = _stage2(lib, ctx, w, scale, limbs, parts=2, out=two).cpu().numpy()
    assert np.array_equal(two, want)


def _round_away(x):
    r = np.trunc(x)
    d = x - r
    return r + (d >= 0.5) - (d <= -0.5)


@pytest.mark.parametrize("chain", ["50", "60/59"])
def test_encode_stage2_rounding_and_reduction(chain):
    """Crafted stage-2 inputs: exact ties (rounded away from zero, as llround), zeros, negatives, and
    coefficients up to 2^60 in magnitude, against the oracle's NTT of round(w * sf) mod q."""

    ctx = _context(chain)
    lib = _bound()
    limbs = 4
    sf = 2.0**20
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    rng = np.random.default_rng(92)
    w = rng.normal(size=(1, N)) * 1000.0
    ties = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.0, -0.0]) / sf
    w[0, :8] = ties
    w[0, 8:16] = np.array([1.0, -1.0, 0.75, -0.75, 1e9, -1e9, 2.0**39.5, -(2.0**39.99)])  # up to 2^60 after sf
    x = _round_away(w[0] * sf)
    coef = np.concatenate([x[0::2], x[1::2]])   # coefficient n < N/2: Re of slot n; n >= N/2: Im of slot n - N/2
    assert np.max(np.abs(coef)) < 2.0**61
    want = np.zeros((limbs, N), dtype=np.uint64)
    for l in range(limbs):
        q = int(ctx.primes[l])
        want[l] = np.array([int(c) % q for c in coef.astype(object)], dtype=np.uint64)
    want = orc.ntt_fwd_limbs(want, list(range(limbs)))
    got = _stage2(lib, ctx, w, sf, limbs).cpu().numpy()[0]
    assert np.array_equal(got, want)


def test_encode_stage2_tables_match_the_library():
    """The exported tables carry the reference's definitions: power_of_roots rows are the
    library's own psi^brv tables, the Shoup companions floor(w 2^64 / p), the per-limb maps the
    Q primes of that limb count then the special primes."""

    ctx = _context("60/59")
    from holmes_amd import _native as nat

    roots = ctx.power_of_roots.cpu().numpy()
    shoup = ctx.power_of_roots_shoup.cpu().numpy()
    assert roots.shape == (ctx.L + ctx.K, N)
    for i in (0, ctx.L - 1, ctx.L + ctx.K - 1):
        host = np.zeros(N, dtype=np.uint64)
        nat.check(nat.lib().hck_context_twiddles(ctx.handle, i, 0, host.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))),
                  "twiddles")
        assert np.array_equal(roots[i], host)
        p = int(ctx.primes[i])
        for k in (0, 1, 12345, N - 1):
            assert int(shoup[i, k]) == (int(roots[i, k]) << 64) // p
    m = ctx.QplusP_map[3].cpu().numpy().tolist()
    assert m == list(ctx.q_primes[:3]) + list(ctx.p_primes)
    diffs = ctx.QmaxdiffplusPmaxdiff_map[3].cpu().numpy().tolist()
    assert diffs == [9223372036854775295 % p for p in m]


def test_encode_stage2_argument_errors():
    ctx = _context("50")
    lib = _bound()
    x = torch.zeros((1, N), dtype=torch.float64, device="cuda")
    out = torch.zeros((1, 2, N), dtype=torch.uint64, device="cuda")
    t = ctx.QplusP_map[2]
    args = [t.data_ptr()] * 4 + [ctx.power_of_roots.data_ptr(), ctx.power_of_roots_shoup.data_ptr(), None, 0, 3, 0]
    assert lib.holmes_encode_stage2(out.data_ptr(), x.data_ptr(), N, 0, 1.0, 2, *args) == 0   # no rows: no-op
    assert lib.holmes_encode_stage2(None, x.data_ptr(), N, 1, 1.0, 2, *args) == -1
    assert lib.holmes_encode_stage2(out.data_ptr(), x.data_ptr(), N, 1, 1.0, 2, None, *args[1:]) == -1
    assert lib.holmes_encode_stage2(out.data_ptr(), x.data_ptr(), 100, 2, 1.0, 2, *args) == -1  # row stride < N
    torch.cuda.synchronize()
