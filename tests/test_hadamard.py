"""Hadamard rotations (holmes_amd.hadamard) against what the mathematics fixes: the Sylvester
matrix in natural order (scipy.linalg.hadamard), H H^T = n I for the order-28 Paley block, the
Kronecker structure the reference's matmul_had_u uses for n = 28 x 512
(tools/convert/hadamard/numpy.py:77-91), and the fuse identity of its down_proj conversion
(tools/convert/hadamard/fuse.py:40-52, 95-112): rotating the activations and the weight's input axis
by the same orthogonal matrix leaves the product unchanged."""

import numpy as np
import pytest
import scipy.linalg

from holmes_amd.hadamard import hadamard_block, hadamard_right, paley2_hadamard, randomized_hadamard_right


def test_paley_block_is_hadamard():
    h = paley2_hadamard(13)
    assert h.shape == (28, 28) and set(np.unique(h)) == {-1, 1}
    assert np.array_equal(h @ h.T, 28 * np.eye(28, dtype=np.int64))
    with pytest.raises(ValueError):
        paley2_hadamard(11)  # 11 = 3 mod 4: the bordered Jacobsthal matrix is not symmetric


@pytest.mark.parametrize("n", [8, 256])
def test_power_of_two_is_sylvester(n):
    rng = np.random.default_rng(n)
    w = rng.normal(size=(5, n))
    want = w @ scipy.linalg.hadamard(n).T / np.sqrt(n)
    assert np.allclose(hadamard_right(w), want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("n", [28 * 4, 28 * 64])
def test_composite_size_is_block_kronecker_sylvester(n):
    rng = np.random.default_rng(n)
    w = rng.normal(size=(3, n))
    block, k = hadamard_block(n)
    assert k == 28
    full = np.kron(block, scipy.linalg.hadamard(n // 28)) / np.sqrt(n)
    assert np.allclose(full @ full.T, np.eye(n), rtol=0, atol=1e-12)
    assert np.allclose(hadamard_right(w), w @ full.T, rtol=0, atol=1e-11)


def test_down_proj_fuse_identity():
    """x_rot @ W^T == x @ W_fused^T with x_rot = x H / sqrt(n) and W_fused = W H / sqrt(n)
    (H symmetric up to the block's transpose: the fused weight uses the same right-rotation)."""

    n = 28 * 16
    rng = np.random.default_rng(7)
    x = rng.normal(size=(4, n))
    w = rng.normal(scale=0.02, size=(6, n))
    x_rot = hadamard_right(x)
    w_fused = hadamard_right(w)
    assert np.allclose(x_rot @ w_fused.T, x @ w.T, rtol=0, atol=1e-12)


def test_randomized_rotation_is_orthogonal_and_seeded():
    n = 28 * 8
    rng = np.random.default_rng(3)
    w = rng.normal(size=(4, n))
    r = randomized_hadamard_right(w, 11)
    assert np.allclose(r @ r.T, w @ w.T, rtol=0, atol=1e-11)  # rows keep their inner products
    assert np.array_equal(r, randomized_hadamard_right(w, 11))
    assert not np.allclose(r, randomized_hadamard_right(w, 12))
    with pytest.raises(ValueError):
        randomized_hadamard_right(np.zeros((2, 24)), 1)
