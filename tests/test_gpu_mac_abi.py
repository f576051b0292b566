"""holmes_mac_multi, the reference sidecar's entry point, called through ctypes with the argtypes the
reference binds (bench/cmp/holmes_multi_mac.py:49) and the argument layout it passes (:129-140):
per-input baby-basis pointers, plaintext rows with a row stride, device arrays of moduli.  Outputs are
bit-exact against the oracle's multiply-accumulate, for 50-bit primes and for the reference's 59/60-bit
chain (assets/feature_major.json: firstMod 60, dcrtBits 59)."""

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
    p, i, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    lib.holmes_mac_multi.argtypes = [p, p, p, ll, i, i, p, ll, i, i, i, p, p, p, p]
    lib.holmes_mac_multi.restype = i
    return lib


@pytest.mark.parametrize("chain", ["50", "60/59"])
def test_holmes_mac_multi_matches_oracle(chain):
    if chain == "50":
        primes = O.gen_primes(16, 50, 4)
    else:
        primes = O.gen_primes(16, 60, 1) + O.gen_primes(16, 59, 3)
    limbs, nb, groups, inputs = 4, 5, 3, 3
    print(f"holmes_mac_multi: chain {chain}, {inputs} inputs, {nb} babies, {groups} groups", flush=True)
    orc = O.OracleContext(16, limbs, 0, 1, primes)
    rng = np.random.default_rng(77)
    q = np.array(primes, dtype=np.uint64).reshape(limbs, 1)

    def residues(*shape):  # [..., limbs (+ padding), N] uniform in [0, q_l), the padding limbs too
        lead, rows = shape[:-2], shape[-2]
        out = rng.integers(0, 1 << 62, size=(*lead, rows, N), dtype=np.uint64)
        out[..., :limbs, :] %= q
        if chain == "60/59":  # edge residues: 0 and q - 1 in the first coefficients
            out[..., :limbs, 0] = 0
            out[..., :limbs, 1] = q[:, 0] - 1
        return out

    pts = residues(groups * nb, limbs + 1, N)          # row stride (limbs + 1) N
    babies = [residues(2, nb, limbs + 2, N) for _ in range(inputs)]  # baby stride (limbs + 2) N
    dev = torch.device("cuda")
    t_pts = torch.from_numpy(pts).to(dev)
    t_c = [(torch.from_numpy(np.ascontiguousarray(b[0])).to(dev), torch.from_numpy(np.ascontiguousarray(b[1])).to(dev))
           for b in babies]
    t_primes = torch.tensor(primes, dtype=torch.uint64, device=dev)
    res = torch.zeros((2, groups, inputs, limbs, N), dtype=torch.uint64, device=dev)
    ptr_t = ctypes.c_void_p * 32
    c0s = ptr_t(*[c0.data_ptr() for c0, _ in t_c])
    c1s = ptr_t(*[c1.data_ptr() for _, c1 in t_c])
    stream = torch.cuda.current_stream().cuda_stream
    lib = _bound()
    code = lib.holmes_mac_multi(res.data_ptr(), c0s, c1s, (limbs + 2) * N, nb, inputs, t_pts.data_ptr(),
                                (limbs + 1) * N, groups, 10108, limbs, t_primes.data_ptr(), None, None, stream)
    assert code == 0
    torch.cuda.synchronize()
    got = res.cpu().numpy()
    for i in range(inputs):
        baby = np.stack([np.stack((babies[i][0][b, :limbs], babies[i][1][b, :limbs])) for b in range(nb)])
        want = orc.bsgs_mac(limbs, nb, groups, pts[:, :limbs], baby)  # [2][G][limbs][N]
        assert np.array_equal(got[:, :, i], want), f"input {i}"


def test_holmes_mac_multi_matches_the_context_mac():
    """The sidecar-shaped entry and hck_bsgs_mac (the one hoisted_mac_sum uses) agree."""

    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=7, dnum=2, seed=3)
    _, ctx = fhe.generate_client_context(spec)
    limbs, nb, groups, inputs = 6, 4, 9, 5
    rng = np.random.default_rng(5)
    q = np.array(ctx.primes[:limbs], dtype=np.uint64).reshape(limbs, 1)
    dev = torch.device("cuda")
    pts = torch.from_numpy(rng.integers(0, 1 << 62, size=(groups * nb, limbs, N), dtype=np.uint64) % q).to(dev)
    base = [torch.from_numpy(rng.integers(0, 1 << 62, size=(nb, inputs, limbs, N), dtype=np.uint64) % q).to(dev)
            for _ in range(2)]
    ref = ctx.bsgs_mac([base[0][b] for b in range(nb)], [base[1][b] for b in range(nb)], pts, limbs, groups)
    # per-input layout: input i's babies [nb][limbs][N] with baby stride inputs * limbs * N
    ptr_t = ctypes.c_void_p * 32
    c0s = ptr_t(*[base[0][0, i].data_ptr() for i in range(inputs)])
    c1s = ptr_t(*[base[1][0, i].data_ptr() for i in range(inputs)])
    res = torch.zeros((2, groups, inputs, limbs, N), dtype=torch.uint64, device=dev)
    lib = _bound()
    # the reference's own call (bench/cmp/holmes_multi_mac.py:138-140): the context's device tables
    # by address, ctx.primes.data_ptr(), ctx.barret_ratio.data_ptr(), ctx.barret_k.data_ptr()
    code = lib.holmes_mac_multi(res.data_ptr(), c0s, c1s, inputs * limbs * N, nb, inputs, pts.data_ptr(), limbs * N,
                                groups, 10116, limbs, ctx.primes.data_ptr(), ctx.barret_ratio.data_ptr(),
                                ctx.barret_k.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    assert torch.equal(res.view(torch.int64).cpu(), ref.view(torch.int64).cpu())


def test_native_context_tables():
    """EasyFHE's context tables with the reference's definitions: primes (Q then P) on the device,
    barret_k = floor(log2 p) + 63, barret_ratio = floor(2^k / p) (bench/cmp/kernels/holmes_mac.cu:56-58),
    PModq = P mod q_i; the Barrett pair reduces products exactly, as the sidecar's barrett128 does."""

    from holmes_amd import fhe

    for dcrt, first in ((50, 50), (59, 60)):
        _, ctx = fhe.generate_client_context(fhe.CKKSContextSpec(depth=5, dnum=2, dcrt_bits=dcrt, first_mod=first,
                                                                 seed=4))
        primes = [int(p) for p in ctx.primes]
        assert torch.tensor(primes, dtype=torch.uint64).tolist() == ctx.primes.tensor.cpu().tolist()
        ratio = [int(v) for v in ctx.barret_ratio.cpu().tolist()]
        k = [int(v) for v in ctx.barret_k.cpu().tolist()]
        P = 1
        for p in ctx.p_primes:
            P *= int(p)
        assert [int(v) for v in ctx.PModq.cpu().tolist()] == [P % int(q) for q in ctx.q_primes]
        rng = np.random.default_rng(dcrt)
        for p, r, kk in zip(primes, ratio, k):
            assert kk == p.bit_length() - 1 + 63 and r == (1 << kk) // p and r < (1 << 64)
            for _ in range(50):
                a, b = (int(x) % p for x in rng.integers(0, 1 << 62, size=2, dtype=np.uint64))
                x = a * b
                est = (x * r) >> kk            # barrett128's quotient estimate
                rem = x - est * p
                while rem >= p:
                    rem -= p
                assert rem == x % p and 0 <= x - est * p < 3 * p
