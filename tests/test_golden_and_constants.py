"""Fixtures vs the oracle, and the product's codec constants vs the fixtures (CPU)."""
import numpy as np
import pytest

from oracle import tq_oracle as O
from kaplumba_amd import codebook as C


def test_oracle_reproduces_codebook_and_sign_fixtures(golden):
    cbs, rots = golden["codebooks"], golden["rotations"]
    for d in (32, 64, 128, 256, 512):
        for b in range(1, 5):
            assert np.array_equal(O.beta_codebook(d, b), cbs[f"beta_{d}_{b}"])
        for seed in (0, 1, 99, 100):
            assert np.array_equal(O.rht_signs(d, seed), rots[f"signs_{d}_{seed}"])
    for b in range(1, 5):
        np.testing.assert_allclose(O.gaussian_lloyd_max(b), cbs[f"gauss_{b}"], rtol=0, atol=1e-14)


def test_oracle_reproduces_quantize_fixtures(golden):
    q = golden["quantize"]
    for d in (32, 64, 128, 256, 512):
        for b in range(1, 5):
            p, n = O.quantize_rht(q[f"x_{d}"], b, O.rht_signs(d, 0), O.beta_codebook(d, b))
            assert np.array_equal(p, q[f"packed_{d}_{b}"])
            assert np.array_equal(n, q[f"norms_{d}_{b}"])


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotation_fixture_matches_recomputation(golden, d):
    for seed in (0, 1):
        np.testing.assert_allclose(O.rotation_matrix(d, seed), golden["rotations"][f"rot_{d}_{seed}"],
                                   rtol=0, atol=1e-6)


def test_product_constants_equal_fixtures(golden):
    """The library's host-side codec constants are the oracle's, bit for bit."""
    cbs, rots = golden["codebooks"], golden["rotations"]
    for d in (32, 64, 128, 256, 512):
        for b in range(1, 5):
            assert np.array_equal(C.beta_codebook(d, b), cbs[f"beta_{d}_{b}"])
            assert np.array_equal(C.midpoints(C.beta_codebook(d, b)), O.midpoints(cbs[f"beta_{d}_{b}"]))
        for seed in (0, 1, 99, 100):
            assert np.array_equal(C.rht_sign_vector(d, seed), rots[f"signs_{d}_{seed}"])
    for b in range(1, 5):
        np.testing.assert_allclose(C.gaussian_levels(b), cbs[f"gauss_{b}"], rtol=0, atol=1e-14)
        assert np.array_equal(C.gaussian_codebook(128, b), O.gaussian_codebook(128, b))
    for d in (64, 128, 256):
        for seed in (0, 1):
            np.testing.assert_allclose(C.rotation_matrix(d, seed), rots[f"rot_{d}_{seed}"], rtol=0, atol=1e-6)
    for d in (64, 96, 128):
        for b in range(1, 5):
            assert C.packed_width(d, b) == O.packed_width(d, b) == (d * b + 31) // 32
